// k_scanf8_bf16.hip -- the ring scans with fp8 (e4m3) logits GEMMs, bf16
// compute dtype.
#include "kernels.hpp"

namespace orda {
ORDA_INSTANTIATE_SCAN_F8(bf16)
}  // namespace orda
