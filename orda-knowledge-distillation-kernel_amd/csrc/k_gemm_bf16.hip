// k_gemm_bf16.hip -- gemm kernels instantiated for bf16 (one object per
// dtype and kernel family so the library builds in parallel).
#include "kernels.hpp"

namespace orda {
ORDA_INSTANTIATE_GEMM(bf16)
}  // namespace orda
