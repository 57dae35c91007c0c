// k_dl_f32.hip -- dl kernels instantiated for float (one object per
// dtype and kernel family so the library builds in parallel).
#include "kernels.hpp"

namespace orda {
ORDA_INSTANTIATE_DL(float)
}  // namespace orda
