// Verify kernel instantiations for bf16 checkpoint state.
#include "verify_kernel.cuh"

namespace gdn {
GDN_DEFINE_VERIFY_LAUNCH(bf16)
}  // namespace gdn
