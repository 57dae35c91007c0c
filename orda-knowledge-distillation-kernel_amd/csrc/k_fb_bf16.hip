// k_fb_bf16.hip -- materialised-path row kernels (in-place dlogits, split-K
// reduce, gradient scaling), instantiated for bf16.
#include "kernels.hpp"

namespace orda {
ORDA_INSTANTIATE_FB(bf16)
}  // namespace orda
