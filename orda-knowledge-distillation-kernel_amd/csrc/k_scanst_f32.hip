// k_scanst_f32.hip -- scan kernels with the logits store (materialised path),
// instantiated for f32.
#include "kernels.hpp"

namespace orda {
ORDA_INSTANTIATE_SCAN_STORE(float)
}  // namespace orda
