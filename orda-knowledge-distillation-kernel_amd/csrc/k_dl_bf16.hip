// k_dl_bf16.hip -- dl kernels instantiated for bf16 (one object per
// dtype and kernel family so the library builds in parallel).
#include "kernels.hpp"

namespace orda {
ORDA_INSTANTIATE_DL(bf16)
}  // namespace orda
