// k_scan_bf16.hip -- scan kernels instantiated for bf16 (one object per
// dtype and kernel family so the library builds in parallel).
#include "kernels.hpp"

namespace orda {
ORDA_INSTANTIATE_SCAN(bf16)
}  // namespace orda
