// Verify kernel instantiations for f16 checkpoint state.
#include "verify_kernel.cuh"

namespace gdn {
GDN_DEFINE_VERIFY_LAUNCH(f16)
}  // namespace gdn
