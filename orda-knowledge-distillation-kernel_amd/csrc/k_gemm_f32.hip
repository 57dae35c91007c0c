// k_gemm_f32.hip -- gemm kernels instantiated for float (one object per
// dtype and kernel family so the library builds in parallel).
#include "kernels.hpp"

namespace orda {
ORDA_INSTANTIATE_GEMM(float)
}  // namespace orda
