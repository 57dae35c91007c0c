// k_fb_f32.hip -- materialised-path row kernels (in-place dlogits, split-K
// reduce, gradient scaling), instantiated for f32.
#include "kernels.hpp"

namespace orda {
ORDA_INSTANTIATE_FB(float)
}  // namespace orda
