// k_scanf8_f16.hip -- the ring scans with fp8 (e4m3) logits GEMMs, fp16
// compute dtype.
#include "kernels.hpp"

namespace orda {
ORDA_INSTANTIATE_SCAN_F8(f16)
}  // namespace orda
