// Verify kernel instantiations for f32 checkpoint state.
#include "verify_kernel.cuh"

namespace gdn {
GDN_DEFINE_VERIFY_LAUNCH(float)
}  // namespace gdn
