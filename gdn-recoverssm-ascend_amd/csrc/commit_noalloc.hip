// The commit for callers that cannot allocate device memory: plan + fold, then
// the conv compaction, with the seven plan arrays in a buffer of this library
// instead of arrays the caller allocates.
//
// The buffer is a file-scope __device__ array, one copy per GPU, alive until
// the process ends. In host code the array's name is a host-side stand-in, not
// a device address, so it is never passed to a kernel or a copy: the first
// call on a device looks up that device's address with hipGetSymbolAddress
// and every launch uses the address kept for the device.
//
// Nothing in the buffer needs clearing: the plan launch stores every entry
// (group < num_groups, row < num_rows) that the fold and the conv compaction
// of the same call read, and both skip a layer mapped to any other group.
#include <mutex>

#include "plan_row.cuh"

namespace gdn {

constexpr int kNoallocPlanes = 7;  // source, lengths, final, boundary, boundary length, valid, column
static __device__ __align__(256) int32_t scratch[kNoallocPlanes * GDN_NOALLOC_PLAN_ENTRIES];

constexpr int kNoallocMaxDevices = 64;
static std::mutex g_noalloc_mu;
static int32_t *g_noalloc_plan[kNoallocMaxDevices];  // device address of `scratch`, per device

// The current device's address of `scratch`, looked up once per device.
static int noalloc_plan_buffer(void *stream, int32_t **out) {
  int dev = -1;
  hipError_t err = hipGetDevice(&dev);
  if (err != hipSuccess || dev < 0 || dev >= kNoallocMaxDevices) {
    set_error("commit_noalloc: no usable current device (%s)", hipGetErrorString(err));
    return GDN_ERR_LAUNCH;
  }
  if (stream) {
    hipDevice_t stream_dev = -1;
    err = hipStreamGetDevice(static_cast<hipStream_t>(stream), &stream_dev);
    if (err != hipSuccess || stream_dev != dev) {
      set_error("commit_noalloc: the stream belongs to device %d, not to the current device %d", int(stream_dev),
                dev);
      return GDN_ERR_INVALID;
    }
  }
  std::lock_guard<std::mutex> lock(g_noalloc_mu);
  if (!g_noalloc_plan[dev]) {
    void *p = nullptr;
    err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess || !p) {
      set_error("commit_noalloc: hipGetSymbolAddress of the plan buffer failed on device %d: %s", dev,
                hipGetErrorString(err));
      return GDN_ERR_LAUNCH;
    }
    g_noalloc_plan[dev] = static_cast<int32_t *>(p);
  }
  *out = g_noalloc_plan[dev];
  return GDN_OK;
}

}  // namespace gdn

using namespace gdn;

extern "C" int gdn_recoverssm_commit_noalloc(const gdn_plan_launch *plan, void *state_ref, const void *correction_ref,
                                             const void *key_ref, const void *decay_ref, const int64_t *state_addrs,
                                             const int64_t *state_block_strides, const int64_t *corr_addrs,
                                             const int64_t *corr_block_strides, const int64_t *key_addrs,
                                             const int64_t *key_block_strides, const int64_t *decay_addrs,
                                             const int64_t *decay_block_strides, const int32_t *layer_groups,
                                             const int64_t *config, int64_t config_len, const gdn_fold_ext *ext,
                                             const gdn_conv_launch *conv, void *stream) {
  if (!plan) {
    set_error("commit_noalloc: missing plan launch block");
    return GDN_ERR_INVALID;
  }
  if (plan->source_plan || plan->lens_plan || plan->final_plan || plan->boundary_plan || plan->boundary_lens_plan ||
      plan->valid_plan || plan->col_plan) {
    set_error("commit_noalloc: the plan arrays are the library's; pass NULL for every plan-array pointer");
    return GDN_ERR_INVALID;
  }
  if (!plan->groups || plan->num_groups < 1 || plan->num_groups > GDN_PLAN_MAX_GROUPS || plan->plan_capacity <= 0 ||
      int64_t(plan->num_groups) * plan->plan_capacity > GDN_NOALLOC_PLAN_ENTRIES) {
    set_error("commit_noalloc: %d groups x plan capacity %lld exceed the library's %d plan entries",
              plan->num_groups, (long long)plan->plan_capacity, GDN_NOALLOC_PLAN_ENTRIES);
    return GDN_ERR_INVALID;
  }
  if (!config || config_len != GDN_FOLD_CONFIG_FIELDS) {
    set_error("commit_noalloc: tiling ABI expects %d config fields", GDN_FOLD_CONFIG_FIELDS);
    return GDN_ERR_INVALID;
  }
  if (ext && ext->row_list) {
    set_error("commit_noalloc: a row list applies to gdn_recoverssm_fold only");
    return GDN_ERR_INVALID;
  }
  const bool grouped = (plan->flags & GDN_PLAN_GROUPED) != 0;
  const gdn_plan_group &g0 = plan->groups[0];
  // The conv compaction reads the plan's source in a grouped commit and the
  // group's state indices otherwise, as the commit with caller-owned arrays.
  const void *conv_source = grouped ? nullptr : g0.state_indices;
  const int32_t conv_source_dtype = grouped ? GDN_DT_I32 : g0.si_dtype;
  const int64_t conv_source_stride = grouped ? 1 : g0.si_stride;
  const int32_t align = (plan->flags & GDN_PLAN_ALIGN) ? 1 : 0;
  const int64_t cap = plan->plan_capacity, layers = config[1], blocks = config[5];

  // Every argument check of both launches runs before the first HIP call.
  // The conv check only tests its plan-array pointers for NULL, so a host
  // placeholder stands in for the device buffer there.
  int st = GDN_OK;
  if (conv) {
    static int32_t placeholder;
    st = conv_compact_launch(conv->conv_addrs, conv->conv_block_strides, conv->conv_dim_strides,
                             conv->conv_token_strides, grouped ? &placeholder : conv_source, conv_source_dtype,
                             conv_source_stride, &placeholder, &placeholder, &placeholder, &placeholder, layer_groups,
                             plan->num_groups, cap, plan->null_block, plan->num_rows, layers, conv->conv_dim,
                             conv->history, conv->window, blocks, conv->element_bytes, align, true, stream);
    if (st != GDN_OK) return st;
  }
  int32_t *buf = nullptr;
  st = noalloc_plan_buffer(stream, &buf);
  if (st != GDN_OK) return st;
  const int64_t n = GDN_NOALLOC_PLAN_ENTRIES;
  gdn_plan_launch L = *plan;
  L.source_plan = buf;
  L.lens_plan = buf + n;
  L.final_plan = buf + 2 * n;
  L.boundary_plan = buf + 3 * n;
  L.boundary_lens_plan = buf + 4 * n;
  L.valid_plan = buf + 5 * n;
  L.col_plan = buf + 6 * n;
  if (grouped) conv_source = L.source_plan;
  st = gdn_recoverssm_plan_fold(&L, state_ref, correction_ref, key_ref, decay_ref, state_addrs, state_block_strides,
                                corr_addrs, corr_block_strides, key_addrs, key_block_strides, decay_addrs,
                                decay_block_strides, layer_groups, config, config_len, ext, stream);
  if (st != GDN_OK || !conv) return st;
  return conv_compact_launch(conv->conv_addrs, conv->conv_block_strides, conv->conv_dim_strides,
                             conv->conv_token_strides, conv_source, conv_source_dtype, conv_source_stride,
                             L.lens_plan, L.final_plan, L.boundary_plan, L.boundary_lens_plan, layer_groups,
                             plan->num_groups, cap, plan->null_block, plan->num_rows, layers, conv->conv_dim,
                             conv->history, conv->window, blocks, conv->element_bytes, align, false, stream);
}
