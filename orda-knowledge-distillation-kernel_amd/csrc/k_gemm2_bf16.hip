// k_gemm2_bf16.hip -- general GEMM (K-major / MN-major operands, split-K),
// instantiated for bf16.
#include "kernels.hpp"

namespace orda {
ORDA_INSTANTIATE_GEMM2(bf16)
}  // namespace orda
