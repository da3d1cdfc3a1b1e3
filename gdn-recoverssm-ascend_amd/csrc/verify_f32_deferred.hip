// Deferred-commit verify kernels (FP32 state): the previous step's fold applied
// inside verify. Instantiated here, apart from the ordinary kernels, so the
// translation units build in parallel.
#include "verify_kernel.cuh"

namespace gdn {

void launch_verify_f32_deferred(int act_dt, int j, int qm, dim3 grid, hipStream_t s, const VerifyArgs &a) {
  switch (act_dt) {
    case GDN_DT_BF16: launch_verify_j<float, bf16, true>(j, qm, grid, s, a); break;
    case GDN_DT_F16: launch_verify_j<float, f16, true>(j, qm, grid, s, a); break;
    default: launch_verify_j<float, float, true>(j, qm, grid, s, a); break;
  }
}

}  // namespace gdn
