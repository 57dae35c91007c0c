// k_dl_f16.hip -- dl kernels instantiated for f16 (one object per
// dtype and kernel family so the library builds in parallel).
#include "kernels.hpp"

namespace orda {
ORDA_INSTANTIATE_DL(f16)
}  // namespace orda
