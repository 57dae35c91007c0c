// k_scanst_bf16.hip -- scan kernels with the logits store (materialised path),
// instantiated for bf16.
#include "kernels.hpp"

namespace orda {
ORDA_INSTANTIATE_SCAN_STORE(bf16)
}  // namespace orda
