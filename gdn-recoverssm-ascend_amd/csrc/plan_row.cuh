// One row of the commit plan (grouped_commit.py:109-222, kernels.py:975-1072),
// shared by the plan kernel and the fold that plans its own rows.
//
// The plan of a (group, row) is a pure function of the step's metadata. It is
// split in two phases so a caller can start streaming the source page as soon
// as the first phase says the row may commit: plan_begin reads the request,
// source page, query offsets, accepted count and computed-token count (all
// independent loads), plan_finish the block-table entries that depend on them.
#pragma once

#include "gdn_common.cuh"

namespace gdn {

struct PlanArgs {
  const void *sampled;
  int64_t sampled_stride, sampled_len;
  int32_t sampled_dtype, num_groups;
  gdn_plan_group groups[GDN_PLAN_MAX_GROUPS];
  int32_t *source, *lens, *final_, *boundary, *boundary_lens, *valid, *col;
  const void *idx_mapping;
  int64_t idx_len;
  int32_t idx_dtype;
  uint32_t flags;
  int32_t *pcols, *pacc;
  int64_t plen, rows, cap, null_block, Q;
};

// Division with truncation toward zero, as the reference kernels' integer `//`.
__device__ __forceinline__ int64_t tdiv(int64_t a, int64_t b) { return a / b; }

struct PlanRow {
  int64_t request, source, bos, eos, count, C;
  bool request_ok, computed_ok;
  int64_t final_idx, boundary, blen, col;
  bool valid;
};

__device__ __forceinline__ PlanRow plan_begin(const PlanArgs &a, const gdn_plan_group &g, int64_t row) {
  const bool align = (a.flags & GDN_PLAN_ALIGN) != 0;
  PlanRow r;
  r.request = g.request_indices ? load_index(g.request_indices, row * g.map_stride, g.map_dtype) : row;
  r.source = load_index(g.state_indices, row * g.si_stride, g.si_dtype);
  r.bos = load_index(g.query_start_loc, row * g.qsl_stride, g.qsl_dtype);
  r.eos = load_index(g.query_start_loc, (row + 1) * g.qsl_stride, g.qsl_dtype);
  const int64_t qlen = r.eos - r.bos;
  r.request_ok = r.request >= 0 && r.request < a.sampled_len;
  if (align) r.request_ok = r.request_ok && r.request < g.table_rows && r.request < g.computed_len;
  const int64_t accepted =
      r.request_ok ? int64_t(int32_t(load_index(a.sampled, r.request * a.sampled_stride, a.sampled_dtype))) : 0;
  int64_t count = min(max(accepted, int64_t(0)), qlen);
  r.count = min(count, a.Q);
  r.C = 0;
  r.computed_ok = true;
  if (align && r.request_ok) {
    r.C = int64_t(int32_t(load_index(g.num_computed, r.request * g.computed_stride, g.computed_dtype)));
    r.computed_ok = r.C >= 0;
  }
  r.final_idx = r.source;
  r.boundary = a.null_block;
  r.blen = 0;
  r.col = 0;
  r.valid = false;
  return r;
}

// Everything `valid` requires except the final page's range.
__device__ __forceinline__ bool plan_may_commit(const PlanArgs &a, const gdn_plan_group &g, const PlanRow &r) {
  const int64_t qlen = r.eos - r.bos;
  const bool geometry = r.bos >= 0 && r.bos <= r.eos && qlen <= a.Q;
  return r.request_ok && geometry && r.source > a.null_block && r.source < g.num_blocks && r.count > 0 &&
         r.count <= qlen && r.computed_ok;
}

__device__ __forceinline__ void plan_finish(const PlanArgs &a, const gdn_plan_group &g, PlanRow &r) {
  const bool align = (a.flags & GDN_PLAN_ALIGN) != 0;
  const bool grouped = (a.flags & GDN_PLAN_GROUPED) != 0;
  const int64_t null_block = a.null_block;
  if (align && r.request_ok) {
    const int64_t position = r.C + r.count;
    r.col = min(tdiv(max(position - 1, int64_t(0)), g.block_size), g.table_width - 1);
    r.final_idx =
        load_index(g.block_table, r.request * g.table_row_stride + r.col * g.table_col_stride, g.table_dtype);
    const int64_t next_boundary = (tdiv(r.C, g.block_size) + 1) * g.block_size;
    const bool crossed = position >= next_boundary;
    r.blen = next_boundary - r.C;
    const int64_t bcol = tdiv(next_boundary, g.block_size) - 1;
    bool load_b = crossed && bcol >= 0 && bcol < g.table_width;
    if (grouped) load_b = load_b && r.computed_ok;
    r.boundary = load_b ? load_index(g.block_table, r.request * g.table_row_stride + bcol * g.table_col_stride,
                                     g.table_dtype)
                        : null_block;
  }
  r.valid = plan_may_commit(a, g, r) && r.final_idx > null_block && r.final_idx < g.num_blocks;
  const bool boundary_ok = r.boundary > null_block && r.boundary < g.num_blocks;
  if (align && !boundary_ok) r.blen = 0;
  if (grouped && !boundary_ok) r.boundary = null_block;
}

// Plan row `row` of every group, its stores and the align publication: the
// body of the plan kernel (one thread per row).
__device__ __forceinline__ void plan_write_row(const PlanArgs &a, int64_t row) {
  const bool align = (a.flags & GDN_PLAN_ALIGN) != 0;
  const int64_t null_block = a.null_block;
  bool all_valid = true;
  int64_t shared_col = -1, shared_request = -1;
  for (int gi = 0; gi < a.num_groups; ++gi) {
    const gdn_plan_group &g = a.groups[gi];
    PlanRow r = plan_begin(a, g, row);
    plan_finish(a, g, r);
    const bool valid = r.valid;
    const int64_t off = int64_t(gi) * a.cap + row;
    if (a.source) a.source[off] = int32_t(valid ? r.source : null_block);
    a.lens[off] = int32_t(valid ? r.count : 0);
    a.final_[off] = int32_t(valid ? r.final_idx : null_block);
    a.boundary[off] = int32_t(valid ? r.boundary : null_block);
    a.boundary_lens[off] = int32_t(valid ? r.blen : 0);
    if (a.valid) a.valid[off] = valid ? 1 : 0;
    if (a.col) a.col[off] = int32_t(r.col);
    if (gi == 0) {
      shared_col = r.col;
      shared_request = r.request;
    } else {
      all_valid = all_valid && r.col == shared_col && r.request == shared_request;
    }
    all_valid = all_valid && valid;
  }
  if ((a.flags & GDN_PLAN_PUBLISH) && align) {
    if (shared_request >= 0 && shared_request < a.idx_len) {
      const int64_t slot = load_index(a.idx_mapping, shared_request, a.idx_dtype);
      if (all_valid && slot >= 0 && slot < a.plen) {
        a.pcols[slot] = int32_t(shared_col);
        a.pacc[slot] = 1;
      }
    }
  }
}

// Host side: validates a plan launch and fills the kernel arguments (defined
// in commit_plan.hip). Returns a GDN_* status with the error message set.
int make_plan_args(const gdn_plan_launch *launch, PlanArgs *out);

// Host side: checks and launches the conv compaction (commit_plan.hip). A
// layer whose group lies outside [0, plan_groups) compacts nothing;
// check_only validates the arguments without launching.
int conv_compact_launch(const int64_t *conv_addrs, const int64_t *conv_block_strides, const int64_t *conv_dim_strides,
                        const int64_t *conv_token_strides, const void *source, int32_t source_dtype,
                        int64_t source_stride, const int32_t *lengths, const int32_t *final_indices,
                        const int32_t *boundary_indices, const int32_t *boundary_lengths,
                        const int32_t *layer_groups, int64_t plan_groups, int64_t plan_capacity, int64_t null_block,
                        int64_t num_rows, int64_t num_layers, int64_t conv_dim, int64_t history, int64_t window,
                        int64_t num_blocks, int32_t element_bytes, int32_t align, bool check_only, void *stream);

}  // namespace gdn
