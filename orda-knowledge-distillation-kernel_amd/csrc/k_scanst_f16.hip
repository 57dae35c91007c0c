// k_scanst_f16.hip -- scan kernels with the logits store (materialised path),
// instantiated for f16.
#include "kernels.hpp"

namespace orda {
ORDA_INSTANTIATE_SCAN_STORE(f16)
}  // namespace orda
