// k_gemm_f16.hip -- gemm kernels instantiated for f16 (one object per
// dtype and kernel family so the library builds in parallel).
#include "kernels.hpp"

namespace orda {
ORDA_INSTANTIATE_GEMM(f16)
}  // namespace orda
