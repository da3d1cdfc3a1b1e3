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

// Whether a request may be read: inside the accepted counts and, in align
// mode, inside the block table and the computed-token counts.
__device__ __forceinline__ bool plan_request_ok(const PlanArgs &a, const gdn_plan_group &g, int64_t request) {
  // Non-short-circuit: the bounds are read together, not behind branches.
  const bool in_align = (request < g.table_rows) & (request < g.computed_len);
  return (request >= 0) & (request < a.sampled_len) & (((a.flags & GDN_PLAN_ALIGN) == 0) | in_align);
}

// The first phase from the words it reads: the row's request, source page
// and query offsets, and the low 32 bits of the request's accepted count and
// computed tokens (the reference narrows both to int32), meaningful only when
// request_ok.
__device__ __forceinline__ PlanRow plan_begin_from(const PlanArgs &a, int64_t request, int64_t source, int64_t bos,
                                                   int64_t eos, bool request_ok, int32_t accepted_lo,
                                                   int32_t computed_lo) {
  const bool align = (a.flags & GDN_PLAN_ALIGN) != 0;
  PlanRow r;
  r.request = request;
  r.source = source;
  r.bos = bos;
  r.eos = eos;
  r.request_ok = request_ok;
  const int64_t accepted = request_ok ? int64_t(accepted_lo) : 0;
  r.count = min(min(max(accepted, int64_t(0)), eos - bos), a.Q);
  r.C = 0;
  r.computed_ok = true;
  if (align && request_ok) {
    r.C = int64_t(computed_lo);
    r.computed_ok = r.C >= 0;
  }
  r.final_idx = r.source;
  r.boundary = a.null_block;
  r.blen = 0;
  r.col = 0;
  r.valid = false;
  return r;
}

__device__ __forceinline__ PlanRow plan_begin(const PlanArgs &a, const gdn_plan_group &g, int64_t row) {
  const int64_t request = g.request_indices ? load_index(g.request_indices, row * g.map_stride, g.map_dtype) : row;
  const bool ok = plan_request_ok(a, g, request);
  const int32_t accepted = ok ? int32_t(load_index(a.sampled, request * a.sampled_stride, a.sampled_dtype)) : 0;
  const int32_t computed = ok && (a.flags & GDN_PLAN_ALIGN)
                               ? int32_t(load_index(g.num_computed, request * g.computed_stride, g.computed_dtype))
                               : 0;
  return plan_begin_from(a, request, load_index(g.state_indices, row * g.si_stride, g.si_dtype),
                         load_index(g.query_start_loc, row * g.qsl_stride, g.qsl_dtype),
                         load_index(g.query_start_loc, (row + 1) * g.qsl_stride, g.qsl_dtype), ok, accepted, computed);
}

// plan_begin for a row that every lane of the wave plans together (the fold's
// workgroups): its words are gathered by one lane-indexed load (lanes 0-7: the
// low and high words of the source page, both query offsets and the request;
// lanes 8-9: the accepted count and computed tokens when the request is the
// row itself), and one more for the accepted count and computed tokens of a
// mapped request. Lanes with nothing to read read the first query offset,
// which is always there. Same values as plan_begin.
//
// plan_lane_addr gives lanes 0-9 their addresses (other lanes keep `addr`),
// so that a caller can gather more words in the same load; plan_from_words
// decodes the gathered word.
__device__ __forceinline__ uintptr_t plan_lane_addr(const PlanArgs &a, const gdn_plan_group &g, int64_t row,
                                                    int lane, uintptr_t addr) {
  // Straight-line on purpose: every address is formed and then selected, so
  // the kernel arguments behind them are read in one batch instead of each
  // behind a branch of its own.
  const bool align = (a.flags & GDN_PLAN_ALIGN) != 0;
  const bool mapped = g.request_indices != nullptr;
  const uintptr_t any = reinterpret_cast<uintptr_t>(g.query_start_loc);
  const bool s64 = g.si_dtype == GDN_DT_I64, q64 = g.qsl_dtype == GDN_DT_I64, m64 = g.map_dtype == GDN_DT_I64;
  const bool a64 = a.sampled_dtype == GDN_DT_I64, c64 = g.computed_dtype == GDN_DT_I64;
  const uintptr_t src = elem_addr(g.state_indices, row * g.si_stride, s64);
  const uintptr_t bos = elem_addr(g.query_start_loc, row * g.qsl_stride, q64);
  const uintptr_t eos = elem_addr(g.query_start_loc, (row + 1) * g.qsl_stride, q64);
  const uintptr_t req_at = elem_addr(g.request_indices, row * g.map_stride, m64);
  const uintptr_t acc_at = elem_addr(a.sampled, row * a.sampled_stride, a64);
  const uintptr_t cmp_at = elem_addr(g.num_computed, row * g.computed_stride, c64);
  const bool row_ok = !mapped & plan_request_ok(a, g, row);
  const uintptr_t req = mapped ? req_at : any;
  const uintptr_t acc = row_ok ? acc_at : any;
  const uintptr_t cmp = row_ok & align ? cmp_at : any;
  addr = lane == 0 ? src : addr;
  addr = lane == 1 ? src + (s64 ? 4 : 0) : addr;
  addr = lane == 2 ? bos : addr;
  addr = lane == 3 ? bos + (q64 ? 4 : 0) : addr;
  addr = lane == 4 ? eos : addr;
  addr = lane == 5 ? eos + (q64 ? 4 : 0) : addr;
  addr = lane == 6 ? req : addr;
  addr = lane == 7 ? req + (mapped & m64 ? 4 : 0) : addr;
  addr = lane == 8 ? acc : addr;
  addr = lane == 9 ? cmp : addr;
  return addr;
}

__device__ __forceinline__ PlanRow plan_from_words(const PlanArgs &a, const gdn_plan_group &g, int64_t row,
                                                   uint32_t w) {
  const bool align = (a.flags & GDN_PLAN_ALIGN) != 0;
  const bool mapped = g.request_indices != nullptr;
  const int lane = int(threadIdx.x & 63);
  const uintptr_t any = reinterpret_cast<uintptr_t>(g.query_start_loc);
  const bool s64 = g.si_dtype == GDN_DT_I64, q64 = g.qsl_dtype == GDN_DT_I64, m64 = g.map_dtype == GDN_DT_I64;
  const bool a64 = a.sampled_dtype == GDN_DT_I64, c64 = g.computed_dtype == GDN_DT_I64;
  const int64_t request = mapped ? index_of(word_of(w, 6), word_of(w, 7), m64) : row;
  int32_t accepted = int32_t(word_of(w, 8)), computed = int32_t(word_of(w, 9));
  const bool ok = plan_request_ok(a, g, request);
  if (mapped) {
    const uintptr_t acc1 = ok ? elem_addr(a.sampled, request * a.sampled_stride, a64) : any;
    const uintptr_t cmp1 = ok && align ? elem_addr(g.num_computed, request * g.computed_stride, c64) : any;
    const uint32_t w1 = lane_word(lane == 0 ? acc1 : cmp1);
    accepted = int32_t(word_of(w1, 0));
    computed = int32_t(word_of(w1, 1));
  }
  return plan_begin_from(a, request, index_of(word_of(w, 0), word_of(w, 1), s64),
                         index_of(word_of(w, 2), word_of(w, 3), q64), index_of(word_of(w, 4), word_of(w, 5), q64), ok,
                         accepted, computed);
}

__device__ __forceinline__ PlanRow plan_begin_lanes(const PlanArgs &a, const gdn_plan_group &g, int64_t row) {
  const int lane = int(threadIdx.x & 63);
  const uintptr_t w = lane_word(plan_lane_addr(a, g, row, lane, reinterpret_cast<uintptr_t>(g.query_start_loc)));
  return plan_from_words(a, g, row, w);
}

// Everything `valid` requires except the final page's range.
__device__ __forceinline__ bool plan_may_commit(const PlanArgs &a, const gdn_plan_group &g, const PlanRow &r) {
  const int64_t qlen = r.eos - r.bos;
  const bool geometry = r.bos >= 0 && r.bos <= r.eos && qlen <= a.Q;
  return r.request_ok && geometry && r.source > a.null_block && r.source < g.num_blocks && r.count > 0 &&
         r.count <= qlen && r.computed_ok;
}

// The second phase's block-table reads: in align mode the final page at the
// column holding the last accepted token and, when the window crosses a block
// boundary, the boundary page; element offsets into the block table.
struct PlanTable {
  bool active, load_b;
  int64_t final_el, boundary_el;
};

__device__ __forceinline__ PlanTable plan_table(const PlanArgs &a, const gdn_plan_group &g, PlanRow &r) {
  PlanTable t{false, false, 0, 0};
  if (!((a.flags & GDN_PLAN_ALIGN) && r.request_ok)) return t;
  const int64_t position = r.C + r.count;
  r.col = min(tdiv(max(position - 1, int64_t(0)), g.block_size), g.table_width - 1);
  const int64_t next_boundary = (tdiv(r.C, g.block_size) + 1) * g.block_size;
  r.blen = next_boundary - r.C;
  const int64_t bcol = tdiv(next_boundary, g.block_size) - 1;
  bool load_b = position >= next_boundary && bcol >= 0 && bcol < g.table_width;
  if (a.flags & GDN_PLAN_GROUPED) load_b = load_b && r.computed_ok;
  t.active = true;
  t.load_b = load_b;
  t.final_el = r.request * g.table_row_stride + r.col * g.table_col_stride;
  t.boundary_el = r.request * g.table_row_stride + bcol * g.table_col_stride;
  return t;
}

// The second phase from the block-table words (used only where plan_table
// asked for them).
__device__ __forceinline__ void plan_finish_from(const PlanArgs &a, const gdn_plan_group &g, PlanRow &r,
                                                 const PlanTable &t, int64_t final_page, int64_t boundary_page) {
  const int64_t null_block = a.null_block;
  if (t.active) {
    r.final_idx = final_page;
    r.boundary = t.load_b ? boundary_page : null_block;
  }
  r.valid = plan_may_commit(a, g, r) && r.final_idx > null_block && r.final_idx < g.num_blocks;
  const bool boundary_ok = r.boundary > null_block && r.boundary < g.num_blocks;
  if ((a.flags & GDN_PLAN_ALIGN) && !boundary_ok) r.blen = 0;
  if ((a.flags & GDN_PLAN_GROUPED) && !boundary_ok) r.boundary = null_block;
}

__device__ __forceinline__ void plan_finish(const PlanArgs &a, const gdn_plan_group &g, PlanRow &r) {
  const PlanTable t = plan_table(a, g, r);
  const int64_t fin = t.active ? load_index_ro(g.block_table, t.final_el, g.table_dtype) : 0;
  const int64_t bnd = t.load_b ? load_index_ro(g.block_table, t.boundary_el, g.table_dtype) : 0;
  plan_finish_from(a, g, r, t, fin, bnd);
}

// plan_finish for a row every lane plans together: both block-table words in
// one lane-indexed load (lanes 0-1 the final page, 2-3 the boundary page).
__device__ __forceinline__ void plan_finish_lanes(const PlanArgs &a, const gdn_plan_group &g, PlanRow &r) {
  const PlanTable t = plan_table(a, g, r);
  int64_t fin = 0, bnd = 0;
  if (t.active) {
    const int lane = int(threadIdx.x & 63);
    const bool t64 = g.table_dtype == GDN_DT_I64;
    const uintptr_t any = reinterpret_cast<uintptr_t>(g.query_start_loc);
    const uintptr_t f = elem_addr(g.block_table, t.final_el, t64);
    const uintptr_t b = t.load_b ? elem_addr(g.block_table, t.boundary_el, t64) : any;
    uintptr_t addr = any;
    addr = lane == 0 ? f : addr;
    addr = lane == 1 ? f + (t64 ? 4 : 0) : addr;
    addr = lane == 2 ? b : addr;
    addr = lane == 3 ? b + (t.load_b && t64 ? 4 : 0) : addr;
    const uint32_t w = lane_word(addr);
    fin = index_of(word_of(w, 0), word_of(w, 1), t64);
    bnd = index_of(word_of(w, 2), word_of(w, 3), t64);
  }
  plan_finish_from(a, g, r, t, fin, bnd);
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
