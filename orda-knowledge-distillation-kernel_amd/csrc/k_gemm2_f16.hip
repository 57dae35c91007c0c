// k_gemm2_f16.hip -- general GEMM (K-major / MN-major operands, split-K),
// instantiated for f16.
#include "kernels.hpp"

namespace orda {
ORDA_INSTANTIATE_GEMM2(f16)
}  // namespace orda
