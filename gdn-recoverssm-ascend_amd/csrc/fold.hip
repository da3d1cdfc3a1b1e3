// Commit fold: replays the accepted prefix of the verify records into each
// layer's checkpoint in place (grouped_commit.py:377-480, kernels.py:1222-1324,
// csrc/fold.h:192-237 of the reference plugin).
//
// One workgroup (256 threads) owns one (layer, row, value head) state [V, K].
// The state is streamed once: each thread loads 16-byte chunks of its rows
// (consecutive threads -> consecutive chunks, so every wave instruction covers
// whole 128-byte lines), folds
//     h <- fma(c_t, k_t, h * decay_t),   t = 0 .. n-1
// in registers, stores the boundary snapshot after `boundary_len` tokens and
// the final state after n tokens. Every chunk a thread stores was loaded by the
// same thread before its first store, so source / final / boundary pages may
// alias. Corrections and keys of the accepted tokens are staged in LDS.
//
// PLANNED (gdn_recoverssm_plan_fold): the workgroup plans its own (group, row)
// instead of reading the plan arrays, issuing the source page's loads as soon
// as the first plan phase allows the row to commit; the first `writers`
// workgroups of the grid store the plan arrays for the conv compaction.
#include "plan_row.cuh"

namespace gdn {

struct FoldArgs {
  const int64_t *state_addrs, *state_bs, *corr_addrs, *corr_bs, *key_addrs, *key_bs, *decay_addrs, *decay_bs;
  const int32_t *layer_groups;
  const void *source;
  const int32_t *lengths, *finals, *boundaries, *boundary_lens;
  int64_t source_stride;
  int64_t rows, heads, ratio, Q, blocks, record_rows, cap, null_block;
  int64_t state_head_stride, state_v_stride;
  int64_t corr_head_stride, corr_token_stride;
  int64_t key_head_stride, key_token_stride;
  int64_t decay_head_stride, decay_token_stride;
  int32_t K, V, KP, KCH;  // KP: K padded to a whole number of chunks; KCH = KP / E
  int32_t kp_log, kch_log;  // KP and KCH are powers of two
  uint32_t v_magic;         // div16_magic(V)
  int32_t source_dtype;
  // Plan rows to fold (unplanned fold only; NULL: rows 0..rows-1): the grid
  // covers grid_rows = row_list_len entries instead of `rows`.
  const int32_t *row_list;
  int64_t grid_rows;
};

constexpr int kFoldThreads = 256;

// State pages move through the fold once (read from the source page, written
// to the final / boundary page, next read by a later step's verify), so both
// directions are non-temporal: they bypass the caches' normal retention and
// leave them to the records. Measured on MI355X this shortens a verify + plan
// + fold step by ~13% against plain loads and stores.
//
// Each (page, head) tile is addressed through a buffer resource covering
// exactly its V rows: a thread keeps one 32-bit offset and the pass step goes
// in the scalar offset, so no per-chunk 64-bit addresses occupy registers
// (four times the occupancy of flat addressing), and rows past V or chunks
// past K read zero and drop their stores without a branch.
typedef unsigned fold_u32x4 __attribute__((ext_vector_type(4)));
constexpr int kFoldNT = 2;                  // buffer cache policy: non-temporal
constexpr int kFoldOutOfRange = 0x7ffff000;  // past any tile's extent (<= 1 MiB)
__device__ __forceinline__ __amdgpu_buffer_rsrc_t fold_tile(const void *p, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), 0, bytes, 0x00020000);
}
__device__ __forceinline__ uint4 load_stream(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
  const fold_u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, kFoldNT);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ void store_stream(__amdgpu_buffer_rsrc_t r, int voff, int soff, const uint4 &x) {
  store_b128_settled<kFoldNT>(gdn_u32x4{x.x, x.y, x.z, x.w}, r, voff, soff);
}

// EARLY: the accepted tokens' corrections and keys are loaded before the state
// tile, so staging them (and the workgroup barrier after it) waits only for
// them, not for the tile behind them in the vector memory counter; for grids
// of a few rounds of workgroups, where each workgroup's critical path shows
// (1.8 us less for the B=64 step's fold; 1.6 us more at B=256, whose launch
// the memory keeps busy anyway). Records of at most one batch.
constexpr int kRecPasses = 4;  // workgroup passes per batch of record loads
constexpr int64_t kEarlyMaxGrid = 4096;

// PACED: in launches of many rounds of workgroups (a commit over every layer
// of a model: 48 layers x 128 rows x 32 heads is ~200k workgroups on 768
// slots) each workgroup waits ~2.5 us (s_sleep 96: 64 x 96 cycles) before its
// state loads. The launch then sustains more bandwidth: the 48-layer commit
// of the decode loop took 3.61-3.63 ms with the wait against 3.76-3.77 ms
// without it, and a workgroup whose planning took one more dependent load (a
// request mapping) gained the same. Fewer workgroups have their 64 KiB load
// bursts queued at once. A launch of a few rounds (a single layer's commit,
// ~8000 workgroups) keeps the immediate order, where each workgroup's latency
// shows (at B=256 one more dependent load before the state loads took the
// plan + fold from 146 to 148.5 us).
constexpr int64_t kPacedMinGrid = 32768;
constexpr int kPaceSleep = 96;
enum FoldOrder : int { kOrderDefault = 0, kOrderEarly = 1, kOrderPaced = 2 };

// The per-layer words a workgroup needs before its first state load: the
// layer's plan group and its tile and record tables (state_addrs, state_bs,
// corr_addrs, corr_bs, key_addrs, key_bs, decay_addrs, decay_bs at the layer).
struct LayerRefs {
  int64_t tab[8];
  int64_t group;
};
// A planning workgroup gathers them with its plan words in one lane-indexed
// load (lane kLayerLane: the group; the next 16 lanes: low and high words of
// the eight tables), so its first state load waits for one round trip after
// the kernel arguments instead of a chain of scalar reads.
constexpr int kLayerLane = 10;
__device__ __forceinline__ uintptr_t layer_lane_addr(const FoldArgs &a, int64_t layer, int lane, uintptr_t addr) {
  const int64_t *const tabs[8] = {a.state_addrs, a.state_bs, a.corr_addrs, a.corr_bs,
                                  a.key_addrs,   a.key_bs,   a.decay_addrs, a.decay_bs};
  addr = (lane == kLayerLane) & (a.layer_groups != nullptr) ? reinterpret_cast<uintptr_t>(a.layer_groups + layer) : addr;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uintptr_t t = reinterpret_cast<uintptr_t>(tabs[i] + layer);
    addr = lane == kLayerLane + 1 + 2 * i ? t : addr;
    addr = lane == kLayerLane + 2 + 2 * i ? t + 4 : addr;
  }
  return addr;
}
__device__ __forceinline__ LayerRefs layer_refs_from(const FoldArgs &a, uint32_t w) {
  LayerRefs L;
#pragma unroll
  for (int i = 0; i < 8; ++i)
    L.tab[i] = index_of(word_of(w, kLayerLane + 1 + 2 * i), word_of(w, kLayerLane + 2 + 2 * i), true);
  L.group = a.layer_groups ? int64_t(int32_t(word_of(w, kLayerLane))) : 0;
  return L;
}
__device__ __forceinline__ LayerRefs layer_refs_load(const FoldArgs &a, int64_t layer) {
  LayerRefs L;
  L.tab[0] = a.state_addrs[layer];
  L.tab[1] = a.state_bs[layer];
  L.tab[2] = a.corr_addrs[layer];
  L.tab[3] = a.corr_bs[layer];
  L.tab[4] = a.key_addrs[layer];
  L.tab[5] = a.key_bs[layer];
  L.tab[6] = a.decay_addrs[layer];
  L.tab[7] = a.decay_bs[layer];
  L.group = a.layer_groups ? int64_t(a.layer_groups[layer]) : 0;
  return L;
}

template <typename S, typename KT, bool PLANNED, int ORDER>
__device__ __forceinline__ void fold_body(const FoldArgs &a, const PlanArgs *p, int64_t w) {
  constexpr int E = Chunk<S>::E;
  constexpr int ITERS = 64 / E;  // chunks held per thread per batch (64 f32 values)
  constexpr bool EARLY = ORDER == kOrderEarly;
  extern __shared__ float lds[];

  // 32-bit division: the grid is below 2^31 workgroups (checked on the host),
  // and a 64-bit division here became a long inline sequence per index.
  const uint32_t wu = uint32_t(w), heads = uint32_t(a.heads), rows = uint32_t(a.grid_rows);
  const int64_t hv = wu % heads;
  int64_t row = (wu / heads) % rows;
  const int64_t layer = wu / (heads * rows);
  if constexpr (!PLANNED) {
    if (a.row_list) {
      // Listed rows: strictly increasing; an entry out of range or not above
      // the one before it folds nothing (a repeated row is folded once).
      const int64_t i = row;
      row = a.row_list[i];
      if (row < 0 || row >= a.rows || (i > 0 && a.row_list[i - 1] >= row)) return;
    }
  }
  int64_t src, fin, bidx;
  int n, blen;
  PlanRow pr;
  LayerRefs L;
  if constexpr (PLANNED) {
    // The values gdn_recoverssm_plan would store for this (group, row), which
    // the fold below reads back under the same checks. A layer mapped to a
    // group the plan does not cover folds nothing. The plan words are
    // gathered for group 0 with the layer's words and gathered again for a
    // layer of another group.
    const gdn_plan_group &g0 = p->groups[0];
    const int lane = int(threadIdx.x & 63);
    uintptr_t addr = layer_lane_addr(a, layer, lane, reinterpret_cast<uintptr_t>(g0.query_start_loc));
    addr = plan_lane_addr(*p, g0, row, lane, addr);
    const uint32_t words = lane_word(addr);
    L = layer_refs_from(a, words);
    const int64_t group = L.group;
    if (group < 0 || group >= p->num_groups) return;
    const gdn_plan_group &g = p->groups[group];
    pr = group == 0 ? plan_from_words(*p, g0, row, words) : plan_begin_lanes(*p, g, row);
    src = pr.source;
    n = int(pr.count);
    if (!(plan_may_commit(*p, g, pr) && src > a.null_block && src < a.blocks && n <= a.Q && row < a.record_rows))
      return;
    fin = bidx = a.null_block;
    blen = 0;
  } else {
    L = layer_refs_load(a, layer);
    const int64_t plan_row = L.group * a.cap + row;
    src = load_index(a.source, plan_row * a.source_stride, a.source_dtype);
    n = a.lengths[plan_row];
    fin = a.finals[plan_row];
    if (!(src > a.null_block && src < a.blocks && n > 0 && n <= a.Q && fin > a.null_block && fin < a.blocks &&
          row < a.record_rows))
      return;
    bidx = a.boundaries[plan_row];
    blen = a.boundary_lens[plan_row];
  }

  S *base = reinterpret_cast<S *>(L.tab[0]);
  const int64_t sbs = L.tab[1];
  const int V = a.V;
  const int64_t vs = a.state_v_stride;
  const int tile_bytes = int(V * vs * int64_t(sizeof(S)));
  const __amdgpu_buffer_rsrc_t rsrc = fold_tile(base + src * sbs + hv * a.state_head_stride, tile_bytes);

  const int tid = threadIdx.x;
  const int KCH = a.KCH;
  const int kc = tid & (KCH - 1);
  const int r0 = tid >> a.kch_log;
  const int RP = kFoldThreads / KCH;  // rows covered by one pass of the workgroup
  const bool kc_ok = kc * E < a.K;
  // Byte offset of the thread's chunk in pass 0 (rows past V fall outside the
  // tile's extent); pass i adds i * step in the scalar offset.
  const int voff = kc_ok ? int((r0 * vs + kc * E) * int64_t(sizeof(S))) : kFoldOutOfRange;
  const int step = int(RP * vs * int64_t(sizeof(S)));

  // Records of the accepted tokens, corrections [n][V] and keys [n][KP] (zero
  // past K), go to LDS. A batch covers kRecPasses passes of the workgroup;
  // its loads are all issued before any is waited for, branch-free (indices
  // past the accepted tokens read as zero). With EARLY the first batch is
  // issued before the state tile, else after it; the host takes EARLY only
  // when one batch holds all the records.
  const float *corr_base = reinterpret_cast<const float *>(L.tab[2]) + row * L.tab[3] + hv * a.corr_head_stride;
  const KT *key_base = reinterpret_cast<const KT *>(L.tab[4]) + row * L.tab[5] + (hv / a.ratio) * a.key_head_stride;
  const __amdgpu_buffer_rsrc_t rcorr = fold_tile(corr_base, kFoldOutOfRange);
  const __amdgpu_buffer_rsrc_t rkey = fold_tile(key_base, kFoldOutOfRange);
  const int n_corr = n * a.V, n_key = n * a.KP;
  auto load_records = [&](int first, float (&c)[kRecPasses], float (&k)[kRecPasses]) {
#pragma unroll
    for (int pp = 0; pp < kRecPasses; ++pp) {
      const int idx = first + pp * kFoldThreads + tid;
      const int t = int(div16(uint32_t(idx), a.v_magic)), v = idx - t * a.V;
      const int coff = idx < n_corr ? int((t * a.corr_token_stride + v) * 4) : kFoldOutOfRange;
      c[pp] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rcorr, coff, 0, 0));
      const int tk = idx >> a.kp_log, kk = idx & (a.KP - 1);
      const int koff = idx < n_key && kk < a.K ? int((tk * a.key_token_stride + kk) * int64_t(sizeof(KT)))
                                               : kFoldOutOfRange;
      if constexpr (sizeof(KT) == 4)
        k[pp] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rkey, koff, 0, 0));
      else
        k[pp] = to_f32(__builtin_bit_cast(KT, (unsigned short)__builtin_amdgcn_raw_buffer_load_b16(rkey, koff, 0, 0)));
    }
  };
  float rec_c[kRecPasses], rec_k[kRecPasses];
  if constexpr (EARLY) load_records(0, rec_c, rec_k);
  if constexpr (ORDER == kOrderPaced) __builtin_amdgcn_s_sleep(kPaceSleep);
  // Issue the first batch of state loads before staging the records.
  uint4 raw[ITERS];
#pragma unroll
  for (int i = 0; i < ITERS; ++i) raw[i] = load_stream(rsrc, voff, i * step);
  if constexpr (PLANNED) {
    const gdn_plan_group &g = p->groups[L.group];
    // Scalar reads: they return on the scalar counter while the state loads
    // above are still in flight (a vector read here would wait for them all).
    plan_finish(*p, g, pr);
    if (!(pr.valid && pr.final_idx > a.null_block && pr.final_idx < a.blocks)) return;
    fin = pr.final_idx;
    bidx = pr.boundary;
    blen = int(pr.blen);
  }
  const bool store_b = bidx > a.null_block && bidx < a.blocks && bidx != fin && blen > 0 && blen <= n;
  const __amdgpu_buffer_rsrc_t rfin = fold_tile(base + fin * sbs + hv * a.state_head_stride, tile_bytes);
  const __amdgpu_buffer_rsrc_t rbnd =
      fold_tile(base + (store_b ? bidx : fin) * sbs + hv * a.state_head_stride, tile_bytes);

  float *corr_lds = lds;                    // [n][V]
  float *key_lds = lds + a.Q * V;           // [n][KP]
  const int KP = a.KP;
  auto stage_records = [&](int first) {
#pragma unroll
    for (int pp = 0; pp < kRecPasses; ++pp) {
      const int idx = first + pp * kFoldThreads + tid;
      if (idx < n_corr) corr_lds[idx] = rec_c[pp];
      if (idx < n_key) key_lds[idx] = rec_k[pp];
    }
  };
  if constexpr (!EARLY) load_records(0, rec_c, rec_k);
  // The first batch is staged outside the loop: staged at a loop header, its
  // waits would be counted for the loop's own loads, issued last, and so
  // would wait for the state tile as well.
  stage_records(0);
  for (int first = kRecPasses * kFoldThreads; first < n_corr || first < n_key; first += kRecPasses * kFoldThreads) {
    load_records(first, rec_c, rec_k);
    stage_records(first);
  }
  // Decays through the scalar path, clamped to the accepted tokens so every
  // read is in bounds (the records are not written while the fold runs).
  // Read as vector loads they would queue behind the state tile.
  const uintptr_t decay_at = reinterpret_cast<uintptr_t>(reinterpret_cast<const float *>(L.tab[6]) + row * L.tab[7] +
                                                          hv * a.decay_head_stride);
  const auto *decay_ro = reinterpret_cast<const __attribute__((address_space(4))) float *>(decay_at);
  float decay[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const float d = decay_ro[(t < n ? t : n - 1) * a.decay_token_stride];
    decay[t] = t < n ? d : 1.0f;
  }
  __syncthreads();

  const int passes = (V + RP - 1) / RP;
  for (int first = 0; first < passes; first += ITERS) {
    if (first > 0) {
#pragma unroll
      for (int i = 0; i < ITERS; ++i) raw[i] = load_stream(rsrc, voff, (first + i) * step);
    }
    float h[ITERS][E];
#pragma unroll
    for (int i = 0; i < ITERS; ++i) unpack16<S>(raw[i], h[i]);
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      if (t < n) {
        float kv[E];
#pragma unroll
        for (int e = 0; e < E; ++e) kv[e] = key_lds[t * KP + kc * E + e];
        const float d = decay[t];
#pragma unroll
        for (int i = 0; i < ITERS; ++i) {
          const int r = r0 + (first + i) * RP;
          const float c = corr_lds[t * V + (r < V ? r : 0)];
#pragma unroll
          for (int e = 0; e < E; ++e) h[i][e] = __builtin_fmaf(c, kv[e], h[i][e] * d);
        }
        if (store_b && t + 1 == blen) {
#pragma unroll
          for (int i = 0; i < ITERS; ++i) store_stream(rbnd, voff, (first + i) * step, pack16<S>(h[i]));
        }
      }
    }
#pragma unroll
    for (int i = 0; i < ITERS; ++i) store_stream(rfin, voff, (first + i) * step, pack16<S>(h[i]));
  }
}

template <typename S, typename KT, int ORDER>
__global__ __launch_bounds__(kFoldThreads) void fold_kernel(FoldArgs a) {
  warm_kernel_args<int(sizeof(FoldArgs))>();
  fold_body<S, KT, false, ORDER>(a, nullptr, blockIdx.x);
}

// The first min(*row_count, grid_rows) entries of the row list, a count the
// device wrote: a fixed grid whose workgroups take the (layer, listed row,
// head) tiles in turn, so a list that the host cannot size costs the tiles it
// names instead of a launch over every row. The count is read through the
// scalar cache (written by an earlier launch, read-only here), so the loop
// bound and every barrier in it are uniform.
template <typename S, typename KT>
__global__ __launch_bounds__(kFoldThreads) void fold_listed_kernel(FoldArgs a, const int32_t *row_count,
                                                                   int64_t layers) {
  warm_kernel_args<int(sizeof(FoldArgs) + sizeof(void *) + sizeof(int64_t))>();
  const auto *count =
      reinterpret_cast<const __attribute__((address_space(4))) int32_t *>(reinterpret_cast<uintptr_t>(row_count));
  const int64_t listed = *count;
  a.grid_rows = listed < 0 ? 0 : listed < a.grid_rows ? listed : a.grid_rows;
  const int64_t tiles = layers * a.grid_rows * a.heads;
  for (int64_t w = blockIdx.x; w < tiles; w += gridDim.x) {
    __syncthreads();  // the previous tile's records in LDS are no longer read
    fold_body<S, KT, false, kOrderDefault>(a, nullptr, w);
  }
}

// The first `writers` workgroups store the plan (one thread per row); the rest
// fold, each planning its own row.
template <typename S, typename KT, int ORDER>
__global__ __launch_bounds__(kFoldThreads) void plan_fold_kernel(FoldArgs a, PlanArgs p, int64_t writers) {
  warm_kernel_args<int(sizeof(FoldArgs) + sizeof(PlanArgs) + sizeof(int64_t))>();
  const int64_t w = blockIdx.x;
  if (w < writers) {
    const int64_t row = w * kFoldThreads + threadIdx.x;
    if (row < p.rows) plan_write_row(p, row);
    return;
  }
  fold_body<S, KT, true, ORDER>(a, &p, w - writers);
}

template <typename S, int ORDER>
static void launch_fold_key(int key_dtype, dim3 grid, size_t lds, hipStream_t s, const FoldArgs &a,
                            const PlanArgs *plan, int64_t writers) {
#define GDN_FOLD_LAUNCH(KT)                                                                                   \
  if (plan)                                                                                                   \
    hipLaunchKernelGGL((plan_fold_kernel<S, KT, ORDER>), grid, dim3(kFoldThreads), lds, s, a, *plan, writers); \
  else                                                                                                        \
    hipLaunchKernelGGL((fold_kernel<S, KT, ORDER>), grid, dim3(kFoldThreads), lds, s, a);
  switch (key_dtype) {
    case GDN_DT_BF16: GDN_FOLD_LAUNCH(bf16) break;
    case GDN_DT_F16: GDN_FOLD_LAUNCH(f16) break;
    default: GDN_FOLD_LAUNCH(float) break;
  }
#undef GDN_FOLD_LAUNCH
}

template <typename S>
static void launch_fold_listed(int key_dtype, dim3 grid, size_t lds, hipStream_t s, const FoldArgs &a,
                               const int32_t *row_count, int64_t layers) {
  switch (key_dtype) {
    case GDN_DT_BF16:
      hipLaunchKernelGGL((fold_listed_kernel<S, bf16>), grid, dim3(kFoldThreads), lds, s, a, row_count, layers);
      break;
    case GDN_DT_F16:
      hipLaunchKernelGGL((fold_listed_kernel<S, f16>), grid, dim3(kFoldThreads), lds, s, a, row_count, layers);
      break;
    default:
      hipLaunchKernelGGL((fold_listed_kernel<S, float>), grid, dim3(kFoldThreads), lds, s, a, row_count, layers);
      break;
  }
}

template <typename S>
static void launch_fold_state(int order, int key_dtype, dim3 grid, size_t lds, hipStream_t s, const FoldArgs &a,
                              const PlanArgs *plan, int64_t writers) {
  switch (order) {
    case kOrderEarly: launch_fold_key<S, kOrderEarly>(key_dtype, grid, lds, s, a, plan, writers); break;
    case kOrderPaced: launch_fold_key<S, kOrderPaced>(key_dtype, grid, lds, s, a, plan, writers); break;
    default: launch_fold_key<S, kOrderDefault>(key_dtype, grid, lds, s, a, plan, writers); break;
  }
}

static bool float_dtype_ok(int32_t dt) { return dt == GDN_DT_F32 || dt == GDN_DT_BF16 || dt == GDN_DT_F16; }

// Checks the fold's configuration and fills the kernel arguments; the plan
// arrays are filled by the caller (the fused entry has none).
static int make_fold_args(const int64_t *state_addrs, const int64_t *state_block_strides, const int64_t *corr_addrs,
                          const int64_t *corr_block_strides, const int64_t *key_addrs,
                          const int64_t *key_block_strides, const int64_t *decay_addrs,
                          const int64_t *decay_block_strides, const int32_t *layer_groups, const int64_t *config,
                          int64_t config_len, const gdn_fold_ext *ext, FoldArgs *out, int64_t *grid, size_t *lds) {
  if (!config || config_len != GDN_FOLD_CONFIG_FIELDS || !ext) {
    set_error("fold: tiling ABI expects %d config fields and an extension block", GDN_FOLD_CONFIG_FIELDS);
    return GDN_ERR_INVALID;
  }
  // Field order of the reference's GDN_FOLD_FIELDS (csrc/common.h:37-54).
  const int64_t rows = config[0], layers = config[1], heads = config[2], key_heads = config[3];
  const int64_t query_len = config[4], blocks = config[5], record_rows = config[6], cap = config[7];
  const int64_t null_block = config[8];
  if (!state_addrs || !state_block_strides || !corr_addrs || !corr_block_strides || !key_addrs ||
      !key_block_strides || !decay_addrs || !decay_block_strides) {
    set_error("fold: missing address table or plan array");
    return GDN_ERR_INVALID;
  }
  if (layers <= 0 || rows <= 0 || rows > record_rows || rows > cap || cap <= 0 || heads <= 0 || key_heads <= 0 ||
      heads % key_heads != 0 || query_len <= 0 || query_len > 8 || blocks <= 0 || null_block < 0) {
    set_error("fold: geometry rows=%lld layers=%lld heads=%lld key_heads=%lld Q=%lld record_rows=%lld cap=%lld",
              (long long)rows, (long long)layers, (long long)heads, (long long)key_heads, (long long)query_len,
              (long long)record_rows, (long long)cap);
    return GDN_ERR_INVALID;
  }
  if (!float_dtype_ok(ext->state_dtype) || !float_dtype_ok(ext->key_dtype)) {
    set_error("fold: unsupported state/key dtype");
    return GDN_ERR_UNSUPPORTED;
  }
  const int E = ext->state_dtype == GDN_DT_F32 ? 4 : 8;
  const int64_t K = ext->key_dim, V = ext->value_dim;
  if (K < 1 || K > 256 || K % E != 0 || V < 1 || V > 1024 || ext->state_k_stride != 1 ||
      config[10] % E != 0 || config[9] % E != 0) {
    set_error("fold: K=%lld V=%lld unsupported (K <= 256 and a multiple of %d, V <= 1024, K contiguous, "
              "16-byte aligned rows)",
              (long long)K, (long long)V, E);
    return GDN_ERR_UNSUPPORTED;
  }
  // A (page, head) tile is addressed as V rows of config[10] elements through
  // one buffer resource: rows must not overlap and the tile must stay far
  // below the out-of-range offset.
  const int64_t tile_bytes = V * config[10] * (E == 4 ? 4 : 2);
  if (config[10] < K || tile_bytes > (int64_t(1) << 27)) {
    set_error("fold: state row stride %lld unsupported (at least K=%lld, tile of V rows <= 128 MiB)",
              (long long)config[10], (long long)K);
    return GDN_ERR_UNSUPPORTED;
  }
  // Record loads take 32-bit offsets from each (row, head)'s first token:
  // the token strides must be non-negative and a window's records must lie
  // far below the out-of-range offset.
  const int64_t key_bytes = ext->key_dtype == GDN_DT_F32 ? 4 : 2;
  const int64_t kp_max = 256;
  if (config[12] < 0 || config[14] < 0 || (query_len * config[12] + V) * 4 >= kFoldOutOfRange ||
      (query_len * config[14] + kp_max) * key_bytes >= kFoldOutOfRange) {
    set_error("fold: record token strides (correction %lld, key %lld) must be non-negative and span under 2 GiB "
              "per window",
              (long long)config[12], (long long)config[14]);
    return GDN_ERR_UNSUPPORTED;
  }
  FoldArgs a{};
  a.state_addrs = state_addrs;
  a.state_bs = state_block_strides;
  a.corr_addrs = corr_addrs;
  a.corr_bs = corr_block_strides;
  a.key_addrs = key_addrs;
  a.key_bs = key_block_strides;
  a.decay_addrs = decay_addrs;
  a.decay_bs = decay_block_strides;
  a.layer_groups = layer_groups;
  a.rows = rows;
  a.heads = heads;
  a.ratio = heads / key_heads;
  a.Q = query_len;
  a.blocks = blocks;
  a.record_rows = record_rows;
  a.cap = cap;
  a.null_block = null_block;
  a.state_head_stride = config[9];
  a.state_v_stride = config[10];
  a.corr_head_stride = config[11];
  a.corr_token_stride = config[12];
  a.key_head_stride = config[13];
  a.key_token_stride = config[14];
  a.decay_head_stride = config[15];
  a.decay_token_stride = config[16];
  a.K = int32_t(K);
  a.V = int32_t(V);
  int kch = 1, kch_log = 0;
  while (kch * E < K) kch *= 2, ++kch_log;
  a.KCH = kch;
  a.KP = kch * E;
  a.kch_log = kch_log;
  a.kp_log = kch_log + (E == 8 ? 3 : E == 4 ? 2 : 1);
  a.v_magic = div16_magic(uint32_t(V));
  a.grid_rows = rows;
  if (ext->row_list) {
    if (ext->row_list_len < 1 || ext->row_list_len > rows) {
      set_error("fold: a row list of %lld entries for %lld rows (1..rows entries)", (long long)ext->row_list_len,
                (long long)rows);
      return GDN_ERR_INVALID;
    }
    a.row_list = ext->row_list;
    a.grid_rows = ext->row_list_len;
  } else if (ext->row_count) {
    set_error("fold: a row count applies to a row list");
    return GDN_ERR_INVALID;
  }
  *out = a;
  *grid = layers * a.grid_rows * heads;
  *lds = size_t(query_len) * size_t(V + a.KP) * sizeof(float);
  return GDN_OK;
}

static int launch_fold(const gdn_fold_ext *ext, int64_t grid, size_t lds, const FoldArgs &a, const PlanArgs *plan,
                       int64_t writers, void *stream) {
  if (grid > 0x7fffffffLL) {
    set_error("fold: grid too large");
    return GDN_ERR_UNSUPPORTED;
  }
  auto s = static_cast<hipStream_t>(stream);
  if (a.row_list && ext->row_count) {
    // The grid loops over the tiles of the listed rows the device counted.
    const int64_t layers = grid / (a.grid_rows * a.heads);
    const dim3 g{unsigned(grid < GDN_FOLD_LISTED_GRID ? grid : GDN_FOLD_LISTED_GRID)};
    switch (ext->state_dtype) {
      case GDN_DT_BF16: launch_fold_listed<bf16>(ext->key_dtype, g, lds, s, a, ext->row_count, layers); break;
      case GDN_DT_F16: launch_fold_listed<f16>(ext->key_dtype, g, lds, s, a, ext->row_count, layers); break;
      default: launch_fold_listed<float>(ext->key_dtype, g, lds, s, a, ext->row_count, layers); break;
    }
    const hipError_t err = hipGetLastError();
    if (err != hipSuccess) {
      set_error("fold: launch failed: %s", hipGetErrorString(err));
      return GDN_ERR_LAUNCH;
    }
    return GDN_OK;
  }
  const dim3 g{unsigned(grid)};
  // Records first for grids of a few rounds, when they fit the early passes.
  // (make_fold_args has checked that every window's records fit 32-bit offsets.)
  const bool early = grid <= kEarlyMaxGrid && a.Q * a.V <= kRecPasses * kFoldThreads &&
                     a.Q * a.KP <= kRecPasses * kFoldThreads;
  const int order = early ? kOrderEarly : grid > kPacedMinGrid ? kOrderPaced : kOrderDefault;
  switch (ext->state_dtype) {
    case GDN_DT_BF16: launch_fold_state<bf16>(order, ext->key_dtype, g, lds, s, a, plan, writers); break;
    case GDN_DT_F16: launch_fold_state<f16>(order, ext->key_dtype, g, lds, s, a, plan, writers); break;
    default: launch_fold_state<float>(order, ext->key_dtype, g, lds, s, a, plan, writers); break;
  }
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error("fold: launch failed: %s", hipGetErrorString(err));
    return GDN_ERR_LAUNCH;
  }
  return GDN_OK;
}

}  // namespace gdn

using namespace gdn;

extern "C" int gdn_recoverssm_fold(void *state_ref, const void *correction_ref, const void *key_ref,
                                   const void *decay_ref, const int64_t *state_addrs,
                                   const int64_t *state_block_strides, const int64_t *corr_addrs,
                                   const int64_t *corr_block_strides, const int64_t *key_addrs,
                                   const int64_t *key_block_strides, const int64_t *decay_addrs,
                                   const int64_t *decay_block_strides, const int32_t *layer_groups,
                                   const void *source, const int32_t *lengths, const int32_t *final_indices,
                                   const int32_t *boundary_indices, const int32_t *boundary_lengths,
                                   const int64_t *config, int64_t config_len, const gdn_fold_ext *ext,
                                   void *stream) {
  (void)state_ref;
  (void)correction_ref;
  (void)key_ref;
  (void)decay_ref;
  FoldArgs a{};
  int64_t grid = 0;
  size_t lds = 0;
  int st = make_fold_args(state_addrs, state_block_strides, corr_addrs, corr_block_strides, key_addrs,
                          key_block_strides, decay_addrs, decay_block_strides, layer_groups, config, config_len, ext,
                          &a, &grid, &lds);
  if (st != GDN_OK) return st;
  if (!source || !lengths || !final_indices || !boundary_indices || !boundary_lengths) {
    set_error("fold: missing address table or plan array");
    return GDN_ERR_INVALID;
  }
  if (ext->source_dtype != GDN_DT_I32 && ext->source_dtype != GDN_DT_I64) {
    set_error("fold: unsupported state/key/source dtype");
    return GDN_ERR_UNSUPPORTED;
  }
  a.source = source;
  a.source_dtype = ext->source_dtype;
  a.source_stride = ext->source_stride;
  a.lengths = lengths;
  a.finals = final_indices;
  a.boundaries = boundary_indices;
  a.boundary_lens = boundary_lengths;
  return launch_fold(ext, grid, lds, a, nullptr, 0, stream);
}

extern "C" int gdn_recoverssm_plan_fold(const gdn_plan_launch *plan, void *state_ref, const void *correction_ref,
                                        const void *key_ref, const void *decay_ref, const int64_t *state_addrs,
                                        const int64_t *state_block_strides, const int64_t *corr_addrs,
                                        const int64_t *corr_block_strides, const int64_t *key_addrs,
                                        const int64_t *key_block_strides, const int64_t *decay_addrs,
                                        const int64_t *decay_block_strides, const int32_t *layer_groups,
                                        const int64_t *config, int64_t config_len, const gdn_fold_ext *ext,
                                        void *stream) {
  (void)state_ref;
  (void)correction_ref;
  (void)key_ref;
  (void)decay_ref;
  PlanArgs p{};
  int st = make_plan_args(plan, &p);
  if (st != GDN_OK) return st;
  FoldArgs a{};
  int64_t grid = 0;
  size_t lds = 0;
  st = make_fold_args(state_addrs, state_block_strides, corr_addrs, corr_block_strides, key_addrs, key_block_strides,
                      decay_addrs, decay_block_strides, layer_groups, config, config_len, ext, &a, &grid, &lds);
  if (st != GDN_OK) return st;
  if (a.row_list) {
    set_error("plan_fold: a row list applies to gdn_recoverssm_fold only");
    return GDN_ERR_INVALID;
  }
  if (a.rows != p.rows || a.cap != p.cap || a.null_block != p.null_block || a.Q != p.Q) {
    set_error("plan_fold: fold rows/capacity/null block/window (%lld/%lld/%lld/%lld) differ from the plan's "
              "(%lld/%lld/%lld/%lld)",
              (long long)a.rows, (long long)a.cap, (long long)a.null_block, (long long)a.Q, (long long)p.rows,
              (long long)p.cap, (long long)p.null_block, (long long)p.Q);
    return GDN_ERR_INVALID;
  }
  // layer_groups is a device table: the kernel skips a layer whose group the
  // plan does not cover.
  const int64_t writers = (p.rows + kFoldThreads - 1) / kFoldThreads;
  return launch_fold(ext, grid + writers, lds, a, &p, writers, stream);
}
