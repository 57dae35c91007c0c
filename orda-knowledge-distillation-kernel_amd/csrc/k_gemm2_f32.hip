// k_gemm2_f32.hip -- general GEMM (K-major / MN-major operands, split-K),
// instantiated for f32.
#include "kernels.hpp"

namespace orda {
ORDA_INSTANTIATE_GEMM2(float)
}  // namespace orda
