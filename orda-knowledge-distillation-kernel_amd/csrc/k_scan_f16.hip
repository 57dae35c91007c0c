// k_scan_f16.hip -- scan kernels instantiated for f16 (one object per
// dtype and kernel family so the library builds in parallel).
#include "kernels.hpp"

namespace orda {
ORDA_INSTANTIATE_SCAN(f16)
}  // namespace orda
