// k_fb_f16.hip -- materialised-path row kernels (in-place dlogits, split-K
// reduce, gradient scaling), instantiated for f16.
#include "kernels.hpp"

namespace orda {
ORDA_INSTANTIATE_FB(f16)
}  // namespace orda
