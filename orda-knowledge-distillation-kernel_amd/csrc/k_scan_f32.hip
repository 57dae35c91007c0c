// k_scan_f32.hip -- scan kernels instantiated for float (one object per
// dtype and kernel family so the library builds in parallel).
#include "kernels.hpp"

namespace orda {
ORDA_INSTANTIATE_SCAN(float)
}  // namespace orda
