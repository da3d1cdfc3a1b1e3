// Commit plan, conv-state compaction and align publication: the integer /
// byte-copy parts of the post-sampling commit. One thread per spec row (plan,
// publication) or per (layer, row, channel) (compaction).
//
// Plan semantics: grouped_commit.py:109-222 (grouped) and kernels.py:975-1072
// (single context). Every index derived from data is bounds-checked against the
// sizes the host passes; an out-of-range index makes the row a no-op (the
// reference would read outside the tensor there).
#include <algorithm>
#include <vector>

#include "plan_row.cuh"

namespace gdn {

__global__ __launch_bounds__(64) void plan_kernel(PlanArgs a) {
  warm_kernel_args<int(sizeof(PlanArgs))>();
  const int64_t row = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (row >= a.rows) return;
  plan_write_row(a, row);
}

// Conv-state compaction. One workgroup per (layer, row, tile of
// kConvChannelsPerThread * 256 channels); thread t handles channels
// tile_base + i*256 + t, so every wave instruction covers consecutive
// channels.
//
// WDW > 0: a channel's window is WDW dwords (<= 16 bytes). When the layer's
// windows are contiguous (token stride 1, dim stride = window, dword-aligned)
// the whole window moves as one 128-bit value: the source window is read once
// for both the final and the boundary history, and each destination window is
// read and written whole, its positions from `history` on carried over
// unchanged, so no written line is left half-written. Other layouts (and
// WDW = 0) use element accesses. All loads of a channel precede its stores, so
// source, final and boundary slots may alias (boundary stored before final, as
// kernels.py:1146-1169).
constexpr int kConvChannelsPerThread = 4;

template <int WDW>
__device__ __forceinline__ unsigned __int128 conv_load_window(const uint32_t *p) {
  unsigned __int128 w = 0;
#pragma unroll
  for (int j = 0; j < WDW; ++j) w |= static_cast<unsigned __int128>(p[j]) << (32 * j);
  return w;
}

template <int WDW>
__device__ __forceinline__ void conv_store_window(uint32_t *p, unsigned __int128 w) {
#pragma unroll
  for (int j = 0; j < WDW; ++j) p[j] = static_cast<uint32_t>(w >> (32 * j));
}

template <typename E, int WDW>
__global__ __launch_bounds__(256) void conv_compact_kernel(
    const int64_t *__restrict__ addrs, const int64_t *__restrict__ block_strides,
    const int64_t *__restrict__ dim_strides, const int64_t *__restrict__ token_strides, const void *source,
    int32_t source_dtype, int64_t source_stride, const int32_t *__restrict__ lengths,
    const int32_t *__restrict__ finals, const int32_t *__restrict__ boundaries,
    const int32_t *__restrict__ boundary_lens, const int32_t *__restrict__ layer_groups, int64_t groups, int64_t cap,
    int64_t null_block, int64_t rows, int64_t conv_dim, int64_t history, int64_t window, int64_t num_blocks,
    int32_t align, int64_t dim_tiles) {
  const int64_t wg = blockIdx.x;
  const int64_t tile = wg % dim_tiles;
  const int64_t row = (wg / dim_tiles) % rows;
  const int64_t layer = wg / (dim_tiles * rows);
  // A layer mapped outside the plan's groups compacts nothing (as the fold
  // folds nothing for it).
  const int64_t group = layer_groups ? int64_t(layer_groups[layer]) : 0;
  if (group < 0 || group >= groups) return;
  const int64_t plan_row = group * cap + row;
  const int64_t src = load_index(source, plan_row * source_stride, source_dtype);
  const int64_t n = lengths[plan_row];
  const int64_t fin = finals[plan_row];
  if (!(src > null_block && src < num_blocks && n >= 1 && n - 1 + history <= window && fin > null_block &&
        fin < num_blocks))
    return;
  int64_t bidx = null_block, blen = 0;
  bool store_b = false;
  if (align) {
    bidx = boundaries[plan_row];
    blen = boundary_lens[plan_row];
    store_b = bidx > null_block && bidx < num_blocks && blen >= 1 && blen - 1 + history <= window;
  }
  // One accepted token kept on its own page: the history already starts at
  // position 0 of the window, so the copy would rewrite every byte unchanged.
  if (n == 1 && fin == src && !store_b) return;
  E *base = reinterpret_cast<E *>(addrs[layer]);
  const int64_t bs = block_strides[layer], ds = dim_strides[layer], ts = token_strides[layer];
  const int64_t c0 = tile * (kConvChannelsPerThread * 256) + threadIdx.x;
  if constexpr (WDW > 0) {
    constexpr int EB = int(sizeof(E));
    if (ts == 1 && ds == window && window * EB == 4 * WDW && (bs * EB) % 4 == 0 &&
        (reinterpret_cast<uintptr_t>(base) & 3u) == 0) {
      const uint32_t *sp = reinterpret_cast<const uint32_t *>(base + src * bs);
      uint32_t *fp = reinterpret_cast<uint32_t *>(base + fin * bs);
      uint32_t *bp = reinterpret_cast<uint32_t *>(base + (store_b ? bidx : fin) * bs);
      const int hbits = int(history) * EB * 8;  // <= 128: history <= window
      const unsigned __int128 hmask =
          hbits >= 128 ? ~static_cast<unsigned __int128>(0) : ((static_cast<unsigned __int128>(1) << hbits) - 1);
      const int fsh = int(n - 1) * EB * 8, bsh = int(blen > 0 ? blen - 1 : 0) * EB * 8;
#pragma unroll
      for (int i = 0; i < kConvChannelsPerThread; ++i) {
        const int64_t c = c0 + int64_t(i) * 256;
        if (c < conv_dim) {
          const unsigned __int128 sw = conv_load_window<WDW>(sp + c * WDW);
          unsigned __int128 fw = conv_load_window<WDW>(fp + c * WDW);
          unsigned __int128 bw = 0;
          if (store_b) bw = conv_load_window<WDW>(bp + c * WDW);
          fw = (fw & ~hmask) | ((sw >> fsh) & hmask);
          if (store_b) {
            bw = (bw & ~hmask) | ((sw >> bsh) & hmask);
            conv_store_window<WDW>(bp + c * WDW, bw);
          }
          conv_store_window<WDW>(fp + c * WDW, fw);
        }
      }
      return;
    }
  }
  constexpr int kMaxHist = 16;
  for (int i = 0; i < kConvChannelsPerThread; ++i) {
    const int64_t d = c0 + int64_t(i) * 256;
    if (d >= conv_dim) break;
    const E *sp = base + src * bs + d * ds;
    E fv[kMaxHist], bv[kMaxHist];
    for (int64_t h = 0; h < history; ++h) fv[h] = sp[(n - 1 + h) * ts];
    if (store_b)
      for (int64_t h = 0; h < history; ++h) bv[h] = sp[(blen - 1 + h) * ts];
    if (store_b) {
      E *bp = base + bidx * bs + d * ds;
      for (int64_t h = 0; h < history; ++h) bp[h * ts] = bv[h];
    }
    E *fp = base + fin * bs + d * ds;
    for (int64_t h = 0; h < history; ++h) fp[h * ts] = fv[h];
  }
}

__global__ __launch_bounds__(64) void publish_kernel(const int64_t *__restrict__ desc, int64_t num_buckets,
                                                     const void *request_indices, int32_t request_dtype,
                                                     int64_t request_stride, const void *idx_mapping,
                                                     int32_t idx_dtype, int64_t idx_len, int32_t *pcols,
                                                     int32_t *pacc, int64_t plen, int64_t rows) {
  const int64_t row = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (row >= rows) return;
  const int32_t *first_cols = reinterpret_cast<const int32_t *>(desc[1]);
  const int32_t shared_col = first_cols[row];
  bool valid = true;
  for (int64_t b = 0; b < num_buckets; ++b) {
    const int32_t *vp = reinterpret_cast<const int32_t *>(desc[4 * b]);
    const int32_t *cp = reinterpret_cast<const int32_t *>(desc[4 * b + 1]);
    const int64_t cap = desc[4 * b + 2];
    const int64_t groups = desc[4 * b + 3];
    for (int64_t g = 0; g < groups; ++g) {
      const int64_t off = g * cap + row;
      valid = valid && vp[off] != 0 && cp[off] == shared_col;
    }
  }
  const int64_t request = load_index(request_indices, row * request_stride, request_dtype);
  if (request < 0 || request >= idx_len) return;
  const int64_t slot = load_index(idx_mapping, request, idx_dtype);
  if (valid && slot >= 0 && slot < plen) {
    pcols[slot] = shared_col;
    pacc[slot] = 1;
  }
}

// What a settle of a deferred commit folds (one workgroup). Pending row r <
// num_rows of group g is applied by the next verify when a next row b of that
// group has rows[b] == r and b's next state index is r's final page (the
// test by which the deferred verify applies a pending commit); the applied
// rows are marked in an LDS bitmap first, so every output entry is then
// written once: 0 for an applied row, the plan's length otherwise. The plan's
// length of every entry handed to the fold becomes 0 (each entry is read and
// written by one thread), so a later settle or flush does not fold it again.
// The rows left with a length in some group are listed in ascending order (a
// prefix sum over each tile of 1024 rows), and their number stored last.
constexpr int kSettleThreads = 1024;
constexpr int kSettleWaves = kSettleThreads / 64;

struct SettleNext {
  const void *si[GDN_SETTLE_MAX_GROUPS];
  int64_t stride[GDN_SETTLE_MAX_GROUPS];
  int64_t rows[GDN_SETTLE_MAX_GROUPS];
  int32_t dtype[GDN_SETTLE_MAX_GROUPS];
};

__global__ __launch_bounds__(kSettleThreads) void settle_kernel(int32_t *__restrict__ lengths,
                                                                const int32_t *__restrict__ finals, int32_t groups,
                                                                int64_t cap, int32_t num_rows,
                                                                const int32_t *__restrict__ rows, SettleNext nx,
                                                                int32_t *__restrict__ out, int32_t *__restrict__ list,
                                                                int32_t *__restrict__ count) {
  constexpr int kWords = GDN_SETTLE_MAX_ROWS / 32;
  __shared__ uint32_t applied[GDN_SETTLE_MAX_GROUPS][kWords];
  __shared__ int32_t wave_count[kSettleWaves];
  const int tid = int(threadIdx.x);
  const int words = (num_rows + 31) / 32;
  for (int g = 0; g < groups; ++g)
    for (int i = tid; i < words; i += kSettleThreads) applied[g][i] = 0u;
  __syncthreads();
  for (int g = 0; g < groups; ++g) {
    for (int64_t b = tid; b < nx.rows[g]; b += kSettleThreads) {
      const int32_t r = rows[b];
      if (r >= 0 && r < num_rows && load_index(nx.si[g], b * nx.stride[g], nx.dtype[g]) == int64_t(finals[g * cap + r]))
        atomicOr(&applied[g][r >> 5], 1u << (r & 31));
    }
  }
  __syncthreads();
  const int lane = tid & 63, wave = tid >> 6;
  int32_t listed = 0;  // rows listed by the tiles before this one (the same in every thread)
  for (int64_t r0 = 0; r0 < cap; r0 += kSettleThreads) {
    const int64_t r = r0 + tid;
    bool left = false;
    if (r < cap) {
      for (int g = 0; g < groups; ++g) {
        const int64_t i = g * cap + r;
        const bool hit = r < num_rows && ((applied[g][r >> 5] >> (r & 31)) & 1u);
        const int32_t n = hit ? 0 : lengths[i];
        out[i] = n;
        if (r < num_rows && n > 0) {
          lengths[i] = 0;  // folded by this settle's fold
          left = true;
        }
      }
    }
    const uint64_t m = __ballot(left);
    if (lane == 0) wave_count[wave] = __popcll(m);
    __syncthreads();
    int32_t before = listed, tile = 0;
    for (int k = 0; k < kSettleWaves; ++k) {
      before += k < wave ? wave_count[k] : 0;
      tile += wave_count[k];
    }
    if (left) list[before + __popcll(m & ((uint64_t(1) << lane) - 1))] = int32_t(r);
    listed += tile;
    __syncthreads();  // wave_count is rewritten by the next tile
  }
  if (tid == 0) *count = listed;
}

static bool index_dtype_ok(int32_t dt) { return dt == GDN_DT_I32 || dt == GDN_DT_I64; }

}  // namespace gdn

using namespace gdn;

namespace gdn {

// Byte range [lo, hi) of the elements a plan launch may touch in one array:
// `n` elements of `esz` bytes at an element stride (empty for a null pointer
// or no element); `n2` / `stride2` add a second dimension (the block table).
struct PlanSpan {
  uintptr_t lo = 0, hi = 0;
  const char *what = "";
};
static PlanSpan plan_span(const char *what, const void *p, int64_t n, int64_t stride, int64_t esz, int64_t n2 = 1,
                          int64_t stride2 = 0) {
  PlanSpan s;
  s.what = what;
  if (!p || n <= 0 || n2 <= 0) return s;
  int64_t lo = 0, hi = 0;  // element offsets of the extreme corners
  for (int64_t a : {int64_t(0), (n - 1) * stride})
    for (int64_t b : {int64_t(0), (n2 - 1) * stride2}) lo = std::min(lo, a + b), hi = std::max(hi, a + b);
  const uintptr_t base = reinterpret_cast<uintptr_t>(p);
  s.lo = base + uintptr_t(lo * esz);
  s.hi = base + uintptr_t((hi + 1) * esz);
  return s;
}
static bool spans_overlap(const PlanSpan &a, const PlanSpan &b) {
  return a.lo < a.hi && b.lo < b.hi && a.lo < b.hi && b.lo < a.hi;
}

// The plan's outputs must not share memory with its inputs or with each
// other: a plan row reads the metadata of other rows (its request's accepted
// count, the block table), and in the fused plan + fold launch the writer
// workgroups store the plan while the folding workgroups plan their rows from
// the same metadata, unordered against them.
static bool plan_memory_disjoint(const gdn_plan_launch *L) {
  const bool align = L->flags & GDN_PLAN_ALIGN;
  auto esz = [](int32_t dt) { return int64_t(dt == GDN_DT_I64 ? 8 : 4); };
  const int64_t rows = L->num_rows, entries = int64_t(L->num_groups) * L->plan_capacity;
  std::vector<PlanSpan> in, outs;
  in.push_back(plan_span("accepted counts", L->sampled, L->sampled_len, L->sampled_stride, esz(L->sampled_dtype)));
  in.push_back(plan_span("request mapping", L->idx_mapping, L->idx_mapping_len, 1, esz(L->idx_mapping_dtype)));
  for (int i = 0; i < L->num_groups; ++i) {
    const gdn_plan_group &g = L->groups[i];
    in.push_back(plan_span("state indices", g.state_indices, rows, g.si_stride, esz(g.si_dtype)));
    in.push_back(plan_span("query offsets", g.query_start_loc, rows + 1, g.qsl_stride, esz(g.qsl_dtype)));
    in.push_back(plan_span("request indices", g.request_indices, rows, g.map_stride, esz(g.map_dtype)));
    if (align) {
      in.push_back(plan_span("block table", g.block_table, g.table_rows, g.table_row_stride, esz(g.table_dtype),
                             g.table_width, g.table_col_stride));
      in.push_back(plan_span("computed tokens", g.num_computed, g.computed_len, g.computed_stride,
                             esz(g.computed_dtype)));
    }
  }
  const int32_t *plan_arrays[7] = {L->source_plan, L->lens_plan,  L->final_plan, L->boundary_plan,
                                   L->boundary_lens_plan, L->valid_plan, L->col_plan};
  for (const int32_t *p : plan_arrays) outs.push_back(plan_span("plan array", p, entries, 1, 4));
  if ((L->flags & GDN_PLAN_PUBLISH) && align) {
    outs.push_back(plan_span("persistent columns", L->persistent_cols, L->persistent_len, 1, 4));
    outs.push_back(plan_span("persistent acceptance", L->persistent_accepted, L->persistent_len, 1, 4));
  }
  for (size_t i = 0; i < outs.size(); ++i) {
    for (const PlanSpan &x : in) {
      if (spans_overlap(outs[i], x)) {
        set_error("plan: a %s output overlaps the %s it reads", outs[i].what, x.what);
        return false;
      }
    }
    for (size_t j = i + 1; j < outs.size(); ++j) {
      if (spans_overlap(outs[i], outs[j])) {
        set_error("plan: two plan outputs (%s, %s) overlap", outs[i].what, outs[j].what);
        return false;
      }
    }
  }
  return true;
}

int make_plan_args(const gdn_plan_launch *L, PlanArgs *out) {
  if (!L) {
    set_error("plan: missing launch block");
    return GDN_ERR_INVALID;
  }
  if (L->num_groups < 1 || L->num_groups > GDN_PLAN_MAX_GROUPS || !L->groups) {
    set_error("plan: num_groups=%d outside [1, %d]", L->num_groups, GDN_PLAN_MAX_GROUPS);
    return GDN_ERR_INVALID;
  }
  if (L->num_rows < 0 || L->num_rows > L->plan_capacity || L->plan_capacity <= 0) {
    set_error("plan: rows=%lld outside plan capacity %lld", (long long)L->num_rows, (long long)L->plan_capacity);
    return GDN_ERR_INVALID;
  }
  if (L->spec_query_len < 1 || L->spec_query_len > 8) {
    set_error("plan: spec_query_len=%lld outside [1, 8]", (long long)L->spec_query_len);
    return GDN_ERR_INVALID;
  }
  if (!L->sampled || !index_dtype_ok(L->sampled_dtype) || L->sampled_len < 0 || !L->lens_plan || !L->final_plan ||
      !L->boundary_plan || !L->boundary_lens_plan) {
    set_error("plan: missing accepted counts or plan outputs");
    return GDN_ERR_INVALID;
  }
  const bool align = L->flags & GDN_PLAN_ALIGN;
  const bool grouped = L->flags & GDN_PLAN_GROUPED;
  if (grouped && !L->source_plan) {
    set_error("plan: grouped plans store the source");
    return GDN_ERR_INVALID;
  }
  if ((L->flags & GDN_PLAN_PUBLISH) && align &&
      (!L->idx_mapping || !L->persistent_cols || !L->persistent_accepted || !index_dtype_ok(L->idx_mapping_dtype))) {
    set_error("plan: publication needs idx_mapping and the persistent outputs");
    return GDN_ERR_INVALID;
  }
  PlanArgs a{};
  a.sampled = L->sampled;
  a.sampled_stride = L->sampled_stride;
  a.sampled_len = L->sampled_len;
  a.sampled_dtype = L->sampled_dtype;
  a.num_groups = L->num_groups;
  for (int i = 0; i < L->num_groups; ++i) {
    const gdn_plan_group &g = L->groups[i];
    if (!g.state_indices || !g.query_start_loc || !index_dtype_ok(g.si_dtype) || !index_dtype_ok(g.qsl_dtype) ||
        (g.request_indices && !index_dtype_ok(g.map_dtype))) {
      set_error("plan: group %d lacks state indices / offsets or has a non-integer dtype", i);
      return GDN_ERR_INVALID;
    }
    if (align && (!g.block_table || !g.num_computed || g.block_size <= 0 || g.table_width <= 0 ||
                  !index_dtype_ok(g.table_dtype) || !index_dtype_ok(g.computed_dtype))) {
      set_error("plan: group %d align metadata incomplete", i);
      return GDN_ERR_INVALID;
    }
    a.groups[i] = g;
  }
  if (!plan_memory_disjoint(L)) return GDN_ERR_INVALID;
  a.source = L->source_plan;
  a.lens = L->lens_plan;
  a.final_ = L->final_plan;
  a.boundary = L->boundary_plan;
  a.boundary_lens = L->boundary_lens_plan;
  a.valid = L->valid_plan;
  a.col = L->col_plan;
  a.idx_mapping = L->idx_mapping;
  a.idx_len = L->idx_mapping ? L->idx_mapping_len : 0;
  a.idx_dtype = L->idx_mapping_dtype;
  a.flags = L->flags;
  a.pcols = L->persistent_cols;
  a.pacc = L->persistent_accepted;
  a.plen = L->persistent_len;
  a.rows = L->num_rows;
  a.cap = L->plan_capacity;
  a.null_block = L->null_block;
  a.Q = L->spec_query_len;
  *out = a;
  return GDN_OK;
}

}  // namespace gdn

extern "C" int gdn_recoverssm_plan(const void *sampled, int32_t sampled_dtype, int64_t sampled_stride,
                                   int64_t sampled_len, const gdn_plan_group *groups, int32_t num_groups,
                                   int32_t *source_plan, int32_t *lens_plan, int32_t *final_plan,
                                   int32_t *boundary_plan, int32_t *boundary_lens_plan, int32_t *valid_plan,
                                   int32_t *col_plan, const void *idx_mapping, int32_t idx_mapping_dtype,
                                   int64_t idx_mapping_len, int32_t *persistent_cols, int32_t *persistent_accepted,
                                   int64_t persistent_len, int64_t num_rows, int64_t plan_capacity,
                                   int64_t null_block, int64_t spec_query_len, uint32_t flags, void *stream) {
  gdn_plan_launch L{};
  L.sampled = sampled;
  L.sampled_stride = sampled_stride;
  L.sampled_len = sampled_len;
  L.sampled_dtype = sampled_dtype;
  L.num_groups = num_groups;
  L.groups = groups;
  L.source_plan = source_plan;
  L.lens_plan = lens_plan;
  L.final_plan = final_plan;
  L.boundary_plan = boundary_plan;
  L.boundary_lens_plan = boundary_lens_plan;
  L.valid_plan = valid_plan;
  L.col_plan = col_plan;
  L.idx_mapping = idx_mapping;
  L.idx_mapping_len = idx_mapping_len;
  L.idx_mapping_dtype = idx_mapping_dtype;
  L.flags = flags;
  L.persistent_cols = persistent_cols;
  L.persistent_accepted = persistent_accepted;
  L.persistent_len = persistent_len;
  L.num_rows = num_rows;
  L.plan_capacity = plan_capacity;
  L.null_block = null_block;
  L.spec_query_len = spec_query_len;
  PlanArgs a{};
  const int st = make_plan_args(&L, &a);
  if (st != GDN_OK) return st;
  if (num_rows == 0) return GDN_OK;
  const unsigned blocks = unsigned((num_rows + 63) / 64);
  hipLaunchKernelGGL(plan_kernel, dim3(blocks), dim3(64), 0, static_cast<hipStream_t>(stream), a);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error("plan: launch failed: %s", hipGetErrorString(err));
    return GDN_ERR_LAUNCH;
  }
  return GDN_OK;
}

namespace gdn {

int conv_compact_launch(const int64_t *conv_addrs, const int64_t *conv_block_strides, const int64_t *conv_dim_strides,
                        const int64_t *conv_token_strides, const void *source, int32_t source_dtype,
                        int64_t source_stride, const int32_t *lengths, const int32_t *final_indices,
                        const int32_t *boundary_indices, const int32_t *boundary_lengths,
                        const int32_t *layer_groups, int64_t plan_groups, int64_t plan_capacity, int64_t null_block,
                        int64_t num_rows, int64_t num_layers, int64_t conv_dim, int64_t history, int64_t window,
                        int64_t num_blocks, int32_t element_bytes, int32_t align, bool check_only, void *stream) {
  if (!conv_addrs || !conv_block_strides || !conv_dim_strides || !conv_token_strides || !source || !lengths ||
      !final_indices || !boundary_indices || !boundary_lengths || !index_dtype_ok(source_dtype)) {
    set_error("conv_compact: missing table or plan pointer");
    return GDN_ERR_INVALID;
  }
  if (history < 1 || history > 16 || window < history || conv_dim < 1 || num_layers < 1 || num_rows < 0) {
    set_error("conv_compact: history=%lld window=%lld dim=%lld layers=%lld unsupported", (long long)history,
              (long long)window, (long long)conv_dim, (long long)num_layers);
    return GDN_ERR_UNSUPPORTED;
  }
  if (element_bytes != 2 && element_bytes != 4) {
    set_error("conv_compact: element size %d unsupported", element_bytes);
    return GDN_ERR_UNSUPPORTED;
  }
  if (num_rows == 0) return GDN_OK;
  const int64_t per_wg = int64_t(kConvChannelsPerThread) * 256;
  const int64_t tiles = (conv_dim + per_wg - 1) / per_wg;
  const int64_t grid = tiles * num_rows * num_layers;
  if (grid > 0x7fffffffLL) {
    set_error("conv_compact: grid too large");
    return GDN_ERR_UNSUPPORTED;
  }
  if (check_only) return GDN_OK;
  auto s = static_cast<hipStream_t>(stream);
  // Dwords per channel window when it fits the 128-bit fast path, else 0.
  const int64_t wbytes = window * element_bytes;
  const int wdw = (wbytes % 4 == 0 && wbytes <= 16) ? int(wbytes / 4) : 0;
#define GDN_CONV_ARGS                                                                                          \
  conv_addrs, conv_block_strides, conv_dim_strides, conv_token_strides, source, source_dtype, source_stride, \
      lengths, final_indices, boundary_indices, boundary_lengths, layer_groups, plan_groups, plan_capacity,   \
      null_block, num_rows, conv_dim, history, window, num_blocks, align, tiles
#define GDN_CONV_LAUNCH(E)                                                                                  \
  switch (wdw) {                                                                                            \
    case 1: hipLaunchKernelGGL((conv_compact_kernel<E, 1>), dim3(unsigned(grid)), dim3(256), 0, s, GDN_CONV_ARGS); break; \
    case 2: hipLaunchKernelGGL((conv_compact_kernel<E, 2>), dim3(unsigned(grid)), dim3(256), 0, s, GDN_CONV_ARGS); break; \
    case 3: hipLaunchKernelGGL((conv_compact_kernel<E, 3>), dim3(unsigned(grid)), dim3(256), 0, s, GDN_CONV_ARGS); break; \
    case 4: hipLaunchKernelGGL((conv_compact_kernel<E, 4>), dim3(unsigned(grid)), dim3(256), 0, s, GDN_CONV_ARGS); break; \
    default: hipLaunchKernelGGL((conv_compact_kernel<E, 0>), dim3(unsigned(grid)), dim3(256), 0, s, GDN_CONV_ARGS); break; \
  }
  if (element_bytes == 2) {
    GDN_CONV_LAUNCH(uint16_t)
  } else {
    GDN_CONV_LAUNCH(uint32_t)
  }
#undef GDN_CONV_LAUNCH
#undef GDN_CONV_ARGS
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error("conv_compact: launch failed: %s", hipGetErrorString(err));
    return GDN_ERR_LAUNCH;
  }
  return GDN_OK;
}

}  // namespace gdn

extern "C" int gdn_recoverssm_conv_compact(const int64_t *conv_addrs, const int64_t *conv_block_strides,
                                           const int64_t *conv_dim_strides, const int64_t *conv_token_strides,
                                           const void *source, int32_t source_dtype, int64_t source_stride,
                                           const int32_t *lengths, const int32_t *final_indices,
                                           const int32_t *boundary_indices, const int32_t *boundary_lengths,
                                           const int32_t *layer_groups, int64_t plan_capacity,
                                           int64_t null_block, int64_t num_rows, int64_t num_layers,
                                           int64_t conv_dim, int64_t history, int64_t window, int64_t num_blocks,
                                           int32_t element_bytes, int32_t align, void *stream) {
  // The caller's plan arrays bound the groups a layer may name.
  return conv_compact_launch(conv_addrs, conv_block_strides, conv_dim_strides, conv_token_strides, source,
                             source_dtype, source_stride, lengths, final_indices, boundary_indices, boundary_lengths,
                             layer_groups, INT64_MAX, plan_capacity, null_block, num_rows, num_layers, conv_dim,
                             history, window, num_blocks, element_bytes, align, false, stream);
}

extern "C" int gdn_recoverssm_publish(const int64_t *descriptors, int64_t num_buckets, const void *request_indices,
                                      int32_t request_dtype, int64_t request_stride, int64_t request_len,
                                      const void *idx_mapping, int32_t idx_mapping_dtype, int64_t idx_mapping_len,
                                      int32_t *persistent_cols, int32_t *persistent_accepted,
                                      int64_t persistent_len, int64_t num_rows, void *stream) {
  if (!descriptors || num_buckets < 1 || !request_indices || !idx_mapping || !persistent_cols ||
      !persistent_accepted || !index_dtype_ok(request_dtype) || !index_dtype_ok(idx_mapping_dtype)) {
    set_error("publish: missing descriptor, mapping or persistent output");
    return GDN_ERR_INVALID;
  }
  if (num_rows < 0 || num_rows > request_len) {
    set_error("publish: rows exceed the request mapping");
    return GDN_ERR_INVALID;
  }
  if (num_rows == 0) return GDN_OK;
  const unsigned blocks = unsigned((num_rows + 63) / 64);
  hipLaunchKernelGGL(publish_kernel, dim3(blocks), dim3(64), 0, static_cast<hipStream_t>(stream), descriptors,
                     num_buckets, request_indices, request_dtype, request_stride, idx_mapping, idx_mapping_dtype,
                     idx_mapping_len, persistent_cols, persistent_accepted, persistent_len, num_rows);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error("publish: launch failed: %s", hipGetErrorString(err));
    return GDN_ERR_LAUNCH;
  }
  return GDN_OK;
}

extern "C" int gdn_recoverssm_settle(int32_t *lengths, const int32_t *finals, int64_t num_groups,
                                     int64_t capacity, int64_t num_rows, const int32_t *rows, int64_t rows_len,
                                     const gdn_settle_next *next, int32_t *out_lengths, int32_t *row_list,
                                     int32_t *row_count, void *stream) {
  if (num_groups < 1 || num_groups > GDN_SETTLE_MAX_GROUPS || capacity < 1 || num_rows < 0 || num_rows > capacity ||
      num_rows > GDN_SETTLE_MAX_ROWS || num_groups * capacity > 0x7fffffffLL) {
    set_error("settle: %lld groups of %lld plan rows with %lld pending rows (1..%d groups, pending rows <= plan "
              "rows and <= %d)",
              (long long)num_groups, (long long)capacity, (long long)num_rows, GDN_SETTLE_MAX_GROUPS,
              GDN_SETTLE_MAX_ROWS);
    return GDN_ERR_INVALID;
  }
  if (!lengths || !finals || !next || !out_lengths || !row_list || !row_count) {
    set_error("settle: missing plan lengths, final pages, next batch, output lengths, row list or count");
    return GDN_ERR_INVALID;
  }
  SettleNext nx{};
  int64_t most = 0;
  for (int64_t g = 0; g < num_groups; ++g) {
    const gdn_settle_next &n = next[g];
    if (n.rows < 0 || (n.rows > 0 && (!n.state_indices || !rows || rows_len < n.rows || !index_dtype_ok(n.dtype) ||
                                      n.stride < 0))) {
      set_error("settle: group %lld: the row map (%lld entries) and the next state indices (int32/int64, stride "
                ">= 0) must cover its %lld next rows",
                (long long)g, (long long)rows_len, (long long)n.rows);
      return GDN_ERR_INVALID;
    }
    nx.si[g] = n.state_indices;
    nx.stride[g] = n.stride;
    nx.rows[g] = n.rows;
    nx.dtype[g] = n.dtype;
    most = std::max(most, n.rows);
  }
  // The outputs are written while the inputs are read: they share memory
  // with no input and with each other (the plan's own lengths stay).
  const int64_t entries = num_groups * capacity;
  const PlanSpan outs[] = {plan_span("output lengths", out_lengths, entries, 1, 4),
                           plan_span("row list", row_list, std::max<int64_t>(num_rows, 1), 1, 4),
                           plan_span("row count", row_count, 1, 1, 4)};
  std::vector<PlanSpan> ins = {plan_span("plan lengths", lengths, entries, 1, 4),
                               plan_span("final pages", finals, entries, 1, 4),
                               plan_span("row map", rows, most, 1, 4)};
  for (int64_t g = 0; g < num_groups; ++g)
    ins.push_back(plan_span("next state indices", next[g].state_indices, next[g].rows, next[g].stride,
                            next[g].dtype == GDN_DT_I64 ? 8 : 4));
  for (size_t i = 0; i < 3; ++i) {
    for (const PlanSpan &x : ins) {
      if (spans_overlap(outs[i], x)) {
        set_error("settle: the %s overlaps the %s", outs[i].what, x.what);
        return GDN_ERR_INVALID;
      }
    }
    for (size_t j = i + 1; j < 3; ++j) {
      if (spans_overlap(outs[i], outs[j])) {
        set_error("settle: the %s overlaps the %s", outs[i].what, outs[j].what);
        return GDN_ERR_INVALID;
      }
    }
  }
  hipLaunchKernelGGL(settle_kernel, dim3(1), dim3(kSettleThreads), 0, static_cast<hipStream_t>(stream), lengths,
                     finals, int32_t(num_groups), capacity, int32_t(num_rows), rows, nx, out_lengths, row_list,
                     row_count);
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error("settle: launch failed: %s", hipGetErrorString(err));
    return GDN_ERR_LAUNCH;
  }
  return GDN_OK;
}
