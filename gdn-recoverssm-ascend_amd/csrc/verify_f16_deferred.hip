// Deferred-commit verify kernels for f16 checkpoint state: the previous
// step's fold applied inside verify. Instantiated apart from the ordinary
// kernels so the translation units build in parallel.
#include "verify_kernel.cuh"

namespace gdn {
GDN_DEFINE_VERIFY_DEFERRED_LAUNCH(f16)
}  // namespace gdn
