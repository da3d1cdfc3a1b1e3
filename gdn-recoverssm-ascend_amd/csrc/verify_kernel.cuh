// Speculative verify of a Gated DeltaNet window from the read-only checkpoint
// (kernels.py:491-697 and csrc/verify.h:284-332 of the reference plugin).
//
// Per (row b, value head hv) the reference advances S <- S*d_t + c_t k_t^T
// token by token. Verify never writes the state back, so this kernel never
// forms S_t: with G_t = d_0 ... d_t,
//     S_{t-1} k_t = G_{t-1} S_0 k_t + sum_{s<t} (G_{t-1}/G_s) (k_s.k_t) c_s
//     S_t q~_t    = G_t     S_0 q~_t + sum_{s<=t} (G_t/G_s)   (k_s.q~_t) c_s
// The state enters only through the 2Q matrix-vector products
// S_0 [k_0 .. k_{Q-1}, q~_0 .. q~_{Q-1}], computed on the matrix cores
// (v_mfma_f32_16x16x4_f32, FP32 in and out) from one read of the state; the
// per-row recurrence then runs on Q-vectors with the Gram matrix
// k_s.{k_t, q~_t}, evaluated incrementally (no divisions):
//     u_j <- d_t u_j + c_t (k_t.k_j),  w_j <- d_t w_j + c_t (k_t.q~_j).
//
// Work decomposition: one wave per (row, value head, 128-row tile of V). The
// tile is eight 16-row MFMA blocks streamed through two register buffers: the
// loads of blocks i+2 and i+3 are in flight while blocks i and i+1 are on the
// matrix cores, and each 64-row half runs its recurrence while the next
// half's loads are outstanding. Everything the recurrence needs from memory
// (v, gates) is loaded before the first state block, because the vector memory
// counter retires in issue order. The deferred-commit variant (DEFER) works
// on 64-row tiles: four blocks, one recurrence.
//
// MFMA operand layout (16x16x4, wave64): A lane l = (row l%16, k-slot l/16),
// B lane l = (k-slot l/16, column l%16), D lane l register r = (row
// 4*(l/16)+r, column l%16). Lane (i, s) holds the 16-byte chunks 4j+s of its
// row, so the k-slot s of MFMA (j, e) holds element E*(4j+s)+e; B uses the
// same permutation of K. Rows read with ordinary loads are loaded in that
// layout; rows read non-temporally (the early rows of a large batch, see
// verify_kernel) are loaded in row runs and reach it through LDS.
//
// Template parameters: S state element type, A activation type (q, k, v and
// the key record / output when they share it), J 16-byte chunks per lane per
// row (K <= 4*E*J), QM window capacity (Q <= QM).
#pragma once

#include "gdn_common.cuh"

namespace gdn {

struct VerifyArgs {
  const void *q, *k, *v, *g, *beta;
  const void *state;
  float *corr;
  void *key;
  float *decay;
  void *out;
  const void *qsl, *indices;
  // Element strides and page counts fit in 32 bits (checked on the host);
  // every product with a row, token or page index is formed in 64 bits.
  int32_t state_bs, q_ts, k_ts, v_ts, g_ts, beta_ts;
  int32_t corr_rs, key_rs, decay_rs, out_ts;
  int32_t qsl_s, idx_s;
  int32_t blocks, null_block;
  int32_t tokens, heads, value_heads, Q, record_rows;
  int32_t state_hs, state_vs;
  int32_t corr_hs, corr_ts, key_hs, key_ts, decay_hs, decay_ts;
  float scale;
  int32_t K, V, NVT;
  int32_t qsl_i64, idx_i64;                  // index dtypes: 1 for int64
  int32_t g_f32, beta_f32, key_f32, out_f32;  // 1: FP32, 0: activation dtype
  int32_t l2norm, key_per_value_head;
  // Fused gating: g and beta hold the raw projections a and b.
  const void *a_log, *dt_bias;
  int32_t gated, a_log_dt, dt_bias_dt;
  float softplus_beta, softplus_threshold;
  // Deferred commit (kernels instantiated with DEFER): for every current row
  // the pending row it continues (p_rows), the previous step's plan arrays
  // indexed by pending row, and that step's records.
  const int32_t *p_rows, *p_src, *p_len, *p_final, *p_bnd, *p_blen;
  const float *p_corr, *p_decay;
  const void *p_key;
  int32_t p_corr_rs, p_key_rs, p_decay_rs;
  int32_t p_corr_hs, p_corr_ts, p_key_hs, p_key_ts, p_decay_hs, p_decay_ts;
  int32_t p_key_f32, p_key_per_value_head, p_record_rows, p_num_rows;
  int32_t nt_rows;  // rows b < nt_rows read their state non-temporally
};

constexpr int kVerifyThreads = 64;  // one wave per (row, value head, tile)
constexpr int kTileRows = 128;     // eight MFMA row blocks of 16 rows
// The deferred-commit kernels stream half tiles: a wave that also stores the
// folded state lives twice as long per row, and with twice as many, shorter
// waves the launch's tail is shorter (measured: 232 against 236 us per step;
// the plain verify is 3 us faster with whole tiles).
constexpr int kDeferTileRows = 64;
// One 16-row block of the state tile on its way from the row-contiguous load
// layout to the matrix-core operand layout: 16 rows x 4J chunks of 16 bytes.
// It is staged in two rounds of half the row's chunks (one for J = 1), so the
// stage holds 16 rows x 2J chunks.
__host__ __device__ constexpr int verify_stage_rounds(int j) { return j >= 2 ? 2 : 1; }
__host__ __device__ constexpr int verify_stage_bytes(int j) { return 16 * (4 * j / verify_stage_rounds(j)) * 16; }
extern __shared__ __align__(16) uint32_t verify_stage[][4];
__host__ __device__ constexpr int verify_tile_rows(bool deferred) { return deferred ? kDeferTileRows : kTileRows; }

typedef float f32x4 __attribute__((ext_vector_type(4)));

template <typename A>
__device__ __forceinline__ float ld_act(const void *p, int64_t i) {
  return to_f32(static_cast<const A *>(p)[i]);
}

template <typename A>
__device__ __forceinline__ void st_f32_or(void *p, int64_t i, bool f32, float x) {
  if (f32)
    static_cast<float *>(p)[i] = x;
  else
    static_cast<A *>(p)[i] = from_f32<A>(x);
}

// Branch-free loads through buffer resources: an invalid lane passes
// kOutOfRange and reads zero, so every load of a phase issues back to back and
// no divergent branch forces a wait on it.
// Resources start at the wave's first token, so every in-bounds offset is far
// below kWindowBytes (the host checks window extents against it).
constexpr int kOutOfRange = 0x7ffff000;
constexpr int kPolicyNT = 2;  // buffer cache policy bit: non-temporal
constexpr int kWindowBytes = 0x7fff0000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *p, int64_t byte_off) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<char *>(static_cast<const char *>(p) + byte_off), 0,
                                           kWindowBytes, 0x00020000);
}

template <typename A>
__device__ __forceinline__ float bits_to_f32(uint32_t u) {
  if constexpr (sizeof(A) == 4)
    return __uint_as_float(u);
  else
    return to_f32(__builtin_bit_cast(A, uint16_t(u)));
}

// One activation element at a byte offset (kOutOfRange reads 0); imm is a
// constant byte displacement applied only to in-range offsets.
template <typename A>
__device__ __forceinline__ float buf_ld_act(__amdgpu_buffer_rsrc_t r, int byte_off, int imm = 0) {
  if constexpr (sizeof(A) == 4)
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, 0));
  else
    return bits_to_f32<A>(__builtin_amdgcn_raw_buffer_load_b16(r, byte_off + imm, 0, 0));
}

// Four consecutive activation elements starting at a byte offset: one 16-byte
// load for FP32 (dword alignment suffices), four 2-byte loads otherwise, which
// need no alignment beyond the element's.
template <typename A>
__device__ __forceinline__ void buf_ld4_act(__amdgpu_buffer_rsrc_t r, int byte_off, float *x) {
  if constexpr (sizeof(A) == 4) {
    const auto u = __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0);
    x[0] = __uint_as_float(u[0]), x[1] = __uint_as_float(u[1]);
    x[2] = __uint_as_float(u[2]), x[3] = __uint_as_float(u[3]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = buf_ld_act<A>(r, byte_off, i * 2);
  }
}

// Wave-uniform 32-bit word through the scalar cache. Only for tensors this
// kernel never writes; the address is rounded down to a dword.
__device__ __forceinline__ uint32_t scalar_word(uintptr_t addr) {
  return *reinterpret_cast<const __attribute__((address_space(4))) uint32_t *>(addr & ~uintptr_t(3));
}

// One per-head parameter (FP32 or 16-bit) through the scalar cache.
template <typename A>
__device__ __forceinline__ float scalar_param(const void *p, int hv, int dt) {
  if (dt == GDN_DT_F32) return __uint_as_float(scalar_word(reinterpret_cast<uintptr_t>(p) + uintptr_t(hv) * 4));
  const uintptr_t addr = reinterpret_cast<uintptr_t>(p) + uintptr_t(hv) * 2;
  const uint32_t w = (scalar_word(addr) >> (int(addr & 2) * 8)) & 0xffffu;
  if (dt == GDN_DT_BF16) return __uint_as_float(w << 16);
  return float(__builtin_bit_cast(f16, uint16_t(w)));
}

template <typename S>
__device__ __forceinline__ float chunk_elem(const uint4 &raw, int e);
template <>
__device__ __forceinline__ float chunk_elem<float>(const uint4 &raw, int e) {
  return __uint_as_float(e == 0 ? raw.x : e == 1 ? raw.y : e == 2 ? raw.z : raw.w);
}
template <>
__device__ __forceinline__ float chunk_elem<bf16>(const uint4 &raw, int e) {
  const uint32_t w = (e >> 1) == 0 ? raw.x : (e >> 1) == 1 ? raw.y : (e >> 1) == 2 ? raw.z : raw.w;
  return __uint_as_float((e & 1) ? (w & 0xffff0000u) : (w << 16));
}
template <>
__device__ __forceinline__ float chunk_elem<f16>(const uint4 &raw, int e) {
  const uint32_t w = (e >> 1) == 0 ? raw.x : (e >> 1) == 1 ? raw.y : (e >> 1) == 2 ? raw.z : raw.w;
  return float(__builtin_bit_cast(f16, uint16_t((e & 1) ? (w >> 16) : (w & 0xffffu))));
}

// Orders the wave's own LDS writes before its later LDS reads. The workgroup
// is a single wave and LDS executes a wave's instructions in order, so no
// s_barrier is needed, and a wave-scope fence does not drain the outstanding
// global loads the way a workgroup barrier's release fence does.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// DEFER: before verifying, apply the previous step's commit for this row (the
// fold of kernels.py:1222-1324, folded into the next verify): the state comes
// from the pending commit's source page, its accepted prefix is replayed from
// the previous step's records block by block, the result is stored to the
// final page (and the boundary snapshot to the boundary page), and the window
// is verified from the folded values, rounded to the state type exactly as
// the stored page is. Each state page is read once per step instead of twice.
// The wave's LDS, declared once per kernel and shared by both cache-policy
// bodies below (a __shared__ array inside each would be allocated twice).
// The non-temporal body also stages state blocks in dynamic LDS
// (verify_stage_bytes), given to the launch only when it has such rows.
template <int QM, int KP, int J, bool DEFER>
struct VerifyLds {
  float m[2 * QM][KP + 4];  // k and q~ vectors, row pitch KP + 4 (bank spread)
  float gram[QM][2 * QM];
  float d[64][2 * QM + 1];  // GEMV results of one 64-row half tile
  float inv[2 * QM];
  __align__(16) float pk[DEFER ? QM : 1][DEFER ? KP : 1];  // pending commit's keys
};

template <typename S, typename A, int J, int QM, bool DEFER, bool NT>
__device__ __forceinline__ void verify_wave(const VerifyArgs &a, VerifyLds<QM, 4 * Chunk<S>::E * J, J, DEFER> &L) {
  constexpr int E = Chunk<S>::E;       // elements per 16-byte chunk
  constexpr int KP = 4 * E * J;        // K padded to 4 k-slots x J chunks x E
  constexpr int NV = 2 * QM;           // used MFMA columns (<= 16)
  constexpr int TILE = verify_tile_rows(DEFER);
  constexpr int NRB = TILE / 16;  // 16-row MFMA blocks per tile (8 or 4)
  auto &m_lds = L.m;
  auto &gram_lds = L.gram;
  auto &d_lds = L.d;
  auto &inv_lds = L.inv;
  auto &pk_lds = L.pk;

  const int nvt = a.NVT;
  const int hv = int(blockIdx.x) / nvt;
  const int vt = int(blockIdx.x) - hv * nvt;
  const int b = int(blockIdx.y);
  const int ratio = a.value_heads / a.heads;
  const int h = hv / ratio;
  const int lane = threadIdx.x;
  const int V = a.V, K = a.K;
  const int row0 = vt * TILE;
  const int Q = a.Q;
  constexpr int AS = int(sizeof(A));

  // ---- 0. the wave's metadata: one lane-indexed load, one wait ----
  // Lanes 0-5: low and high words of query_start_loc[b], query_start_loc[b+1]
  // and state_indices[b]; DEFER: lane 6 the pending row of b.
  int64_t bos, eos, slot;
  int prow = 0;
  {
    const uintptr_t q0 = elem_addr(a.qsl, int64_t(b) * a.qsl_s, a.qsl_i64);
    const uintptr_t q1 = elem_addr(a.qsl, int64_t(b + 1) * a.qsl_s, a.qsl_i64);
    const uintptr_t s0 = elem_addr(a.indices, int64_t(b) * a.idx_s, a.idx_i64);
    const uintptr_t hq = a.qsl_i64 ? 4 : 0, hs = a.idx_i64 ? 4 : 0;
    uintptr_t addr = q0;
    addr = lane == 1 ? q0 + hq : addr;
    addr = lane == 2 ? q1 : addr;
    addr = lane == 3 ? q1 + hq : addr;
    addr = lane == 4 ? s0 : addr;
    addr = lane == 5 ? s0 + hs : addr;
    if constexpr (DEFER) addr = lane == 6 ? reinterpret_cast<uintptr_t>(a.p_rows) + uintptr_t(b) * 4u : addr;
    const uint32_t w = lane_word(addr);
    bos = index_of(word_of(w, 0), word_of(w, 1), a.qsl_i64);
    eos = index_of(word_of(w, 2), word_of(w, 3), a.qsl_i64);
    slot = index_of(word_of(w, 4), word_of(w, 5), a.idx_i64);
    if constexpr (DEFER) prow = int(word_of(w, 6));
  }
  const int64_t qlen = eos - bos;
  const int64_t out_base = int64_t(hv) * V + row0;
  // Token validity is uniform across the wave (kernels.py:612): lane t < QM
  // tests token t and one ballot gathers the window's mask (an unrolled test
  // per token became a chain of scalar branches).
  uint32_t valid_mask;
  {
    const int64_t tok = bos + lane;
    const bool tv = lane < QM && lane < Q && lane < qlen && tok >= 0 && tok < a.tokens;
    valid_mask = uint32_t(__builtin_amdgcn_ballot_w64(tv));
  }

  // ---- 1. gates (and DEFER: the pending plan and decays): one load ----
  // Lane t < QM reads the dword holding g of token t, lane QM + t that of
  // beta (FP32, or the 16-bit value at its half); every address is formed on
  // its own lane. Tokens outside the window read the first word of
  // query_start_loc (always present; g and beta may be empty, hence null,
  // when the launch has no token at all) and are discarded. DEFER: lanes
  // 2QM .. 2QM+4 read the pending row's accepted length, source, final and
  // boundary pages and boundary length, and lanes 2QM+5 .. 3QM+4 its decays;
  // a row without a pending row reads row 0 (num_rows >= 1) and discards it.
  // The ordinary kernel waits for these words only after its state loads
  // issue; the deferred one needs the pending source page first.
  const int gsz = a.g_f32 ? 4 : AS, bsz = a.beta_f32 ? 4 : AS;
  const uintptr_t any_word = reinterpret_cast<uintptr_t>(a.qsl);
  const bool gate_lane_b = lane >= QM;          // lanes QM .. 2QM-1 carry beta
  const int gate_t = (gate_lane_b ? lane - QM : lane) & 31;
  int gate_sh;                                   // bit offset of this lane's 16-bit gate in its word
  uint32_t gw;
  const bool prow_ok = DEFER && prow >= 0 && prow < a.p_num_rows && prow < a.p_record_rows;
  const int pr = prow_ok ? prow : 0;
  {
    const bool tv = lane < 2 * QM && ((valid_mask >> gate_t) & 1u);
    const uintptr_t base = reinterpret_cast<uintptr_t>(gate_lane_b ? a.beta : a.g);
    const int64_t ts = gate_lane_b ? a.beta_ts : a.g_ts;
    const int64_t sz = gate_lane_b ? bsz : gsz;
    uintptr_t addr = tv ? base + uintptr_t(((bos + gate_t) * ts + hv) * sz) : any_word;
    gate_sh = int(addr & 2) * 8;
    if constexpr (DEFER) {
      const int32_t *plan[5] = {a.p_len, a.p_src, a.p_final, a.p_bnd, a.p_blen};
#pragma unroll
      for (int i = 0; i < 5; ++i)
        addr = lane == 2 * QM + i ? reinterpret_cast<uintptr_t>(plan[i] + pr) : addr;
      const int dt = lane - (2 * QM + 5);
      const uintptr_t da = reinterpret_cast<uintptr_t>(a.p_decay) +
                           uintptr_t((int64_t(pr) * a.p_decay_rs + int64_t(hv) * a.p_decay_hs +
                                      int64_t(dt) * a.p_decay_ts) * 4);
      addr = dt >= 0 && dt < QM ? (dt < Q ? da : any_word) : addr;
    }
    gw = lane_word(addr & ~uintptr_t(3));
  }

  // Pending commit of the previous step (same validity rule as the fold,
  // kernels.py:1232-1242 / csrc/fold.h:192-205). The row continues pending
  // row `prow` (plan and record row of the previous step) only when its state
  // index names that commit's final page: a row whose request is new, or
  // whose metadata names another page, verifies from its own page and leaves
  // the pending commit to a flush.
  bool pend = false, pstore_b = false;
  int pn = 0, pblen = 0;
  int64_t psrc = 0, pfin = 0, pbnd = 0;
  if constexpr (DEFER) {
    pn = int(word_of(gw, 2 * QM + 0));
    psrc = int(word_of(gw, 2 * QM + 1));
    pfin = int(word_of(gw, 2 * QM + 2));
    pbnd = int(word_of(gw, 2 * QM + 3));
    pblen = int(word_of(gw, 2 * QM + 4));
    pend = prow_ok && pn > 0 && pn <= Q && psrc > a.null_block && psrc < a.blocks && pfin > a.null_block &&
           pfin < a.blocks && pfin == slot;
    pstore_b = pend && pbnd > a.null_block && pbnd < a.blocks && pbnd != pfin && pblen > 0 && pblen <= pn;
    prow = pend ? prow : 0;  // record addressing below stays inside the records
  }
  const int pend_len = pend ? pn : 0;  // tokens of the pending commit to replay
  const bool null_slot = slot <= a.null_block || slot >= a.blocks;
  if (null_slot) {
    // Null or out-of-range page: zero outputs for the window, records untouched
    // (kernels.py:569-583).
    for (int t = 0; t < Q; ++t) {
      const int64_t tok = bos + t;
      if (!(t < qlen && tok >= 0 && tok < a.tokens)) continue;
      for (int r = lane; r < TILE; r += kVerifyThreads)
        if (row0 + r < V) st_f32_or<A>(a.out, tok * a.out_ts + out_base + r, a.out_f32 != 0, 0.0f);
    }
    return;  // a pending commit needs slot == its final page, never a null one
  }
  if (valid_mask == 0 && !pend) return;
  // A pending commit on a row with nothing to verify still has to be applied:
  // that wave runs the whole pipeline with no token (every input load reads
  // out of range and nothing but the folded tile is stored).
  const bool verify_row = !null_slot && valid_mask != 0;
  if (!verify_row) valid_mask = 0;

  const int li = lane & 15, ls = lane >> 4;  // MFMA row / column index and k-slot

  // ---- 2. small loads first: k/q chunks, v of the lane's rows ----
  constexpr int C4 = KP / 4;  // 4-element chunks per vector
  constexpr int STAGE_PASSES = (NV * C4 + kVerifyThreads - 1) / kVerifyThreads;
  // DEFER: the pending commit's keys (token t, element kk) for LDS, FP32 or
  // activation-typed records (one of the two loads reads out of range).
  constexpr int PK_PASSES = DEFER ? (QM * C4 + kVerifyThreads - 1) / kVerifyThreads : 1;
  float pkx[PK_PASSES][4];
  if constexpr (DEFER) {
    const int key_head = a.p_key_per_value_head ? hv : h;
    const int64_t kbase = int64_t(prow) * a.p_key_rs + int64_t(key_head) * a.p_key_hs;
    const bool kf32 = a.p_key_f32 != 0;
    const __amdgpu_buffer_rsrc_t rpk = make_rsrc(a.p_key, kbase * (kf32 ? 4 : AS));
    int lim = pend_len;
    asm volatile("" : "+v"(lim));  // per-lane select, not a branch (see load_block)
#pragma unroll
    for (int p = 0; p < PK_PASSES; ++p) {
      const int idx = p * kVerifyThreads + lane;
      const int t = idx / C4, kk = (idx - t * C4) * 4;
      const bool live = t < lim && kk < K;
      const int el = t * a.p_key_ts + kk;
      float x32[4], xa[4];
      buf_ld4_act<float>(rpk, live && kf32 ? el * 4 : kOutOfRange, x32);
      buf_ld4_act<A>(rpk, live && !kf32 ? el * AS : kOutOfRange, xa);
#pragma unroll
      for (int e = 0; e < 4; ++e) pkx[p][e] = x32[e] + xa[e];
    }
  }
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(a.q, bos * a.q_ts * AS), rk = make_rsrc(a.k, bos * a.k_ts * AS);
  float xs[STAGE_PASSES][4];
#pragma unroll
  for (int p = 0; p < STAGE_PASSES; ++p) {
    const int idx = p * kVerifyThreads + lane;
    const int vid = idx / C4, kk = (idx - vid * C4) * 4;
    const bool is_q = vid >= QM;
    const int t = (is_q ? vid - QM : vid) & 31;
    // Non-short-circuit tests: a short-circuit chain became a branch per pass,
    // with kernel arguments reloaded inside it.
    const bool live = (vid < NV) & (((valid_mask >> t) & 1u) != 0) & (kk < K);
    const int el = t * (is_q ? a.q_ts : a.k_ts) + h * K + kk;
    const int off = live ? el * AS : kOutOfRange;
    if constexpr (C4 * QM % kVerifyThreads == 0) {
      // Every pass lies wholly inside the k vectors or wholly inside the q ones.
      buf_ld4_act<A>(p * kVerifyThreads < C4 * QM ? rk : rq, off, xs[p]);
    } else {
      float xq[4], xk[4];
      buf_ld4_act<A>(rq, is_q ? off : kOutOfRange, xq);
      buf_ld4_act<A>(rk, is_q ? kOutOfRange : off, xk);
#pragma unroll
      for (int e = 0; e < 4; ++e) xs[p][e] = xq[e] + xk[e];
    }
  }
  // v of the lane's row in each half; the second half is loaded later, after
  // the loads it must not wait behind.
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(a.v, bos * a.v_ts * AS);
  float vv[2][QM];
  auto load_v = [&](int half) {
#pragma unroll
    for (int t = 0; t < QM; ++t) {
      const int vr = row0 + half * 64 + lane;
      const bool ok = (vr < V) & (((valid_mask >> t) & 1u) != 0);
      const int off = ok ? (t * int(a.v_ts) + int(out_base) + half * 64 + lane) * AS : kOutOfRange;
      vv[half][t] = buf_ld_act<A>(rv, off);
    }
  };
  load_v(0);

  // ---- 3. first two state blocks ----
  // Buffer loads: one resource per (slot, head) tile and a 32-bit per-lane
  // offset per chunk. Rows >= V lie past the resource's extent and read as
  // zero; chunks >= K get an out-of-range offset.
  // Ordinary loads (NT false) read the operand layout directly: load j of
  // block rb gives lane (li, ls) chunk 4j + ls of row rb*16 + li, 16 rows x
  // 64 bytes per load. Non-temporal loads that touch half of each of 16 lines
  // fetched lines twice and ran slower than ordinary ones (131 against 116 us
  // for the B=256 tiles alone), so the non-temporal body (NT) reads rows in
  // long runs: a block is 16 rows x CPR 16-byte chunks (CPR = 4J, the padded
  // row), staged through LDS into the operand layout in ROUNDS rounds of SC =
  // CPR / ROUNDS chunks per row (`transpose` below; with ordinary loads that
  // detour cost 4 us). Load j belongs to round g = j / JR and gives lane l the
  // chunk (row (j % JR)*RPL + l/SC, chunk g*SC + l%SC): 4 rows x 256 bytes per
  // load at K = 128 FP32 (whole rows measured 102 us for the same tiles, runs
  // of 256 bytes 104 us, and halving the stage keeps the LDS from limiting
  // the waves per CU).
  const int tile_rows = V - row0 < TILE ? V - row0 : TILE;
  const int tile_bytes = tile_rows * a.state_vs * int(sizeof(S));
  auto tile_rsrc = [&](int64_t page, bool use) {
    const S *tp = static_cast<const S *>(a.state) + page * a.state_bs + int64_t(hv) * a.state_hs +
                  int64_t(row0) * a.state_vs;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<S *>(use ? tp : static_cast<const S *>(a.state)), 0,
                                             use ? tile_bytes : 0, 0x00020000);
  };
  // DEFER with a pending commit: read the pending source page; the folded
  // tile goes to the final page (and its snapshot to the boundary page).
  const __amdgpu_buffer_rsrc_t rsrc = tile_rsrc(pend ? psrc : slot, true);
  const __amdgpu_buffer_rsrc_t rfin = tile_rsrc(pfin, pend);
  const __amdgpu_buffer_rsrc_t rbnd = tile_rsrc(pbnd, pstore_b);
  const int row_bytes = a.state_vs * int(sizeof(S));
  // A 24-bit product (row_bytes < 2^24, checked on the host): a full multiply
  // here became a 64-bit multiply-add whose unused high addend was a register
  // with a load in flight, and waiting for it held back the first state loads.
  const int lane_off = int(__umul24(unsigned(li), unsigned(row_bytes))) + ls * 16;
  constexpr int CPR = 4 * J;                 // 16-byte chunks per padded row (J <= 16)
  constexpr int ROUNDS = verify_stage_rounds(J);
  constexpr int SC = CPR / ROUNDS;           // chunks of each row staged per round
  constexpr int JR = J / ROUNDS;             // loads (and operand registers) per round
  constexpr int RPL = 64 / SC;               // rows per load
  const int c_chunk = lane & (SC - 1), c_row = lane / SC;
  const int c_off = int(__umul24(unsigned(c_row), unsigned(row_bytes))) + c_chunk * 16;
  const int load_step = RPL * row_bytes;
  // Lane offset of load j (its round's chunks past K read and write nothing)
  // and the uniform part that rides in soffset.
  auto c_voff = [&](int j) { return ((j / JR) * SC + c_chunk) * E < K ? c_off : kOutOfRange; };
  auto c_soff = [&](int rb, int j) { return rb * 16 * row_bytes + (j % JR) * load_step + (j / JR) * SC * 16; };
  // The pending corrections of the lane's row, fetched with each block.
  const __amdgpu_buffer_rsrc_t rpc =
      make_rsrc(a.p_corr, (int64_t(prow) * a.p_corr_rs + int64_t(hv) * a.p_corr_hs + row0) * 4);
  // One form for every K, and every block is loaded (blocks past V read as
  // zero): a conditional load would leave a path on which it was not issued,
  // and the wait counts of every later MFMA would have to assume that path,
  // draining the pipeline at each block.
  auto load_block = [&](int rb, uint4 (&dst)[J], float (&pc)[QM]) {
    // The block step rides in soffset, which the range check covers as well.
#pragma unroll
    for (int j = 0; j < J; ++j) {
      if constexpr (NT) {
        dst[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, c_voff(j), c_soff(rb, j), kPolicyNT));
      } else {
        const int vo = (4 * j + ls) * E < K ? lane_off + j * 64 : kOutOfRange;
        dst[j] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, vo, rb * 16 * row_bytes, 0));
      }
    }
    if constexpr (DEFER) {
      const int v = rb * 16 + li;
      // Tokens to replay as a per-lane value: a select on it stays a select
      // (a wave-uniform bound would turn each load into a branch).
      int lim = row0 + v < V ? pend_len : 0;
      asm volatile("" : "+v"(lim));
#pragma unroll
      for (int t = 0; t < QM; ++t)
        pc[t] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
            rpc, t < lim ? (t * a.p_corr_ts + v) * 4 : kOutOfRange, 0, 0));
    }
  };
  // Row-run block -> operand layout through LDS, one round at a time. In a
  // round, chunk c (of the round's SC) of block row r sits at r*SC +
  // (c ^ swz(r)): the 64 lanes of a write cover 64 consecutive slots, and the
  // 16 lanes (li = 0..15) of a read that share ls hit 16 distinct 16-byte
  // bank groups. Operand register j (chunk 4j + ls) belongs to round j / JR.
  constexpr int SWZ_MASK = (SC < 16 ? SC : 16) - 1;
  constexpr int SWZ_SH = SC >= 16 ? 0 : SC == 8 ? 1 : 2;
  auto swz = [](int r) { return (r >> SWZ_SH) & SWZ_MASK; };
  auto row_slot = [&](int j) {  // slot of load j's chunk
    const int r = (j % JR) * RPL + c_row;
    return r * SC + (c_chunk ^ swz(r));
  };
  auto op_slot = [&](int j) { return li * SC + ((4 * (j % JR) + ls) ^ swz(li)); };  // slot of operand register j
  auto stage_write = [&](const uint4 (&buf)[J], int g) {
#pragma unroll
    for (int j = g * JR; j < (g + 1) * JR; ++j) *reinterpret_cast<uint4 *>(verify_stage[row_slot(j)]) = buf[j];
  };
  auto stage_read = [&](uint4 (&buf)[J], int g) {
#pragma unroll
    for (int j = g * JR; j < (g + 1) * JR; ++j) buf[j] = *reinterpret_cast<const uint4 *>(verify_stage[op_slot(j)]);
  };
  auto transpose = [&](uint4 (&buf)[J]) {
    if constexpr (NT) {
#pragma unroll
      for (int g = 0; g < ROUNDS; ++g) {
        stage_write(buf, g);
        wave_lds_sync();
        stage_read(buf, g);
        wave_lds_sync();  // the next round's writes stay behind these reads
      }
    }
  };
  uint4 bufA[J], bufB[J];
  float pcA[QM], pcB[QM];
  load_block(0, bufA, pcA);
  __builtin_amdgcn_sched_barrier(0);  // keep block 0's loads ahead of block 1's
  load_block(1, bufB, pcB);
  float dec[QM], bet[QM];
  float neg_a = 0.0f, dtb = 0.0f;
  if (a.gated) {
    neg_a = -expf(scalar_param<A>(a.a_log, hv, a.a_log_dt));
    dtb = scalar_param<A>(a.dt_bias, hv, a.dt_bias_dt);
  }
  {
    // Each gate lane decodes its own word; the window's decays and betas then
    // reach every lane by readlane.
    const bool f32 = gate_lane_b ? a.beta_f32 != 0 : a.g_f32 != 0;
    float x = f32 ? __uint_as_float(gw) : bits_to_f32<A>((gw >> gate_sh) & 0xffffu);
    if (a.gated) {
      // docs/reference/recoverssm_gdn_upstream.py:135-151
      if (gate_lane_b) {
        x = 1.0f / (1.0f + expf(-x));
      } else {
        const float xb = x + dtb;
        const float bx = a.softplus_beta * xb;
        const float sp = bx <= a.softplus_threshold ? log1pf(expf(bx)) / a.softplus_beta : xb;
        x = neg_a * sp;
      }
    }
    const float gate = gate_lane_b ? x : expf(x);
#pragma unroll
    for (int t = 0; t < QM; ++t) {
      const bool tv = (valid_mask >> t) & 1u;
      dec[t] = tv ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gate), t)) : 1.0f;
      bet[t] = tv ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gate), QM + t)) : 0.0f;
    }
  }

  // ---- 4. stage vectors and records ----
  const bool rec_ok = b < a.record_rows;
  const bool key_writer = rec_ok && vt == 0 && (a.key_per_value_head || (hv % ratio) == 0);
  const int key_head = a.key_per_value_head ? hv : h;
  const bool key_f32 = a.key_f32 != 0;
#pragma unroll
  for (int p = 0; p < STAGE_PASSES; ++p) {
    const int idx = p * kVerifyThreads + lane;
    const int vid = idx / C4, kk = (idx - vid * C4) * 4;
    if (vid < NV) {
      const bool is_q = vid >= QM;
      const float sc = (is_q && !a.l2norm) ? a.scale : 1.0f;
#pragma unroll
      for (int e = 0; e < 4; ++e) m_lds[vid][kk + e] = xs[p][e] * sc;
      const int t = is_q ? vid - QM : vid;
      if (!is_q && !a.l2norm && key_writer && ((valid_mask >> t) & 1u) && kk < K) {
        const int64_t base = int64_t(b) * a.key_rs + int64_t(key_head) * a.key_hs + int64_t(t) * a.key_ts + kk;
#pragma unroll
        for (int e = 0; e < 4; ++e) st_f32_or<A>(a.key, base + e, key_f32, xs[p][e]);
      }
    }
  }
  if (rec_ok && vt == 0) {
    float dl = 1.0f;
#pragma unroll
    for (int t = 0; t < QM; ++t) dl = lane == t ? dec[t] : dl;
    if (lane < QM && ((valid_mask >> lane) & 1u))
      a.decay[int64_t(b) * a.decay_rs + int64_t(hv) * a.decay_hs + int64_t(lane) * a.decay_ts] = dl;
  }
  // DEFER: the pending keys to LDS, the pending decays to scalars.
  float pdec[QM];
  if constexpr (DEFER) {
#pragma unroll
    for (int p = 0; p < PK_PASSES; ++p) {
      const int idx = p * kVerifyThreads + lane;
      const int t = idx / C4, kk = (idx - t * C4) * 4;
      if (t < QM) {
#pragma unroll
        for (int e = 0; e < 4; ++e) pk_lds[t][kk + e] = pkx[p][e];
      }
    }
#pragma unroll
    for (int t = 0; t < QM; ++t) {
      const bool live = pend && t < pn;
      pdec[t] = live ? __uint_as_float(word_of(gw, 2 * QM + 5 + t)) : 1.0f;
    }
  }
  wave_lds_sync();

  // DEFER: replay the pending accepted prefix on one block in registers,
  // h <- fma(c_t, k_t, h * d_t) as the fold does, storing the boundary snapshot
  // after `boundary_len` tokens and the final state after n (kernels.py:1242-1324).
  // The final store is issued on every path (an unused one falls out of
  // range) so the wait counts of the loads in flight do not depend on the row.
  // The boundary snapshot's store, with its two LDS rounds, only runs on rows
  // that have one (about one tile in seven at B=256): skipping the round trip
  // elsewhere took the 48-layer deferred loop from 5.37-5.46 to 5.32 ms per
  // step, which outweighs the stricter waits on the snapshot rows.
  auto fold_block = [&](int rb, uint4 (&buf)[J], const float (&pc)[QM]) {
    if constexpr (DEFER) {
      const int seg = pstore_b ? pblen : 0;
      // FP32 values of the lane's chunks; the fold keeps them in FP32 across
      // the boundary snapshot and rounds only what it stores, as the fold does.
      float h[J][E];
#pragma unroll
      for (int j = 0; j < J; ++j) unpack16<S>(buf[j], h[j]);
      auto apply = [&](int lo, int hi) {
#pragma unroll
        for (int t = 0; t < QM; ++t) {
          if (t >= lo && t < hi) {
            const float d = pdec[t], c = pc[t];
#pragma unroll
            for (int j = 0; j < J; ++j) {
#pragma unroll
              for (int e4 = 0; e4 < E; e4 += 4) {
                const float4 kv = *reinterpret_cast<const float4 *>(&pk_lds[t][E * (4 * j + ls) + e4]);
                h[j][e4 + 0] = __builtin_fmaf(c, kv.x, h[j][e4 + 0] * d);
                h[j][e4 + 1] = __builtin_fmaf(c, kv.y, h[j][e4 + 1] * d);
                h[j][e4 + 2] = __builtin_fmaf(c, kv.z, h[j][e4 + 2] * d);
                h[j][e4 + 3] = __builtin_fmaf(c, kv.w, h[j][e4 + 3] * d);
              }
            }
          }
        }
      };
      auto store = [&](__amdgpu_buffer_rsrc_t r) {
        if constexpr (NT) {
          // Row runs, non-temporal: the folded chunks go back through LDS
          // into the load layout (each lane writes the slots it read its
          // operands from). Stores of 64-byte pieces of 16 rows ran slower,
          // and non-temporal ones much slower: a synthetic twin of this
          // launch's traffic took 224 us with the operand-layout stores and
          // 192 us with whole-row non-temporal ones.
#pragma unroll
          for (int g = 0; g < ROUNDS; ++g) {
#pragma unroll
            for (int j = g * JR; j < (g + 1) * JR; ++j)
              *reinterpret_cast<uint4 *>(verify_stage[op_slot(j)]) = pack16<S>(h[j]);
            wave_lds_sync();
            // The round's row runs are read back first, then stored: each
            // store's wait then holds back only the stores behind it.
            uint4 x[JR];
#pragma unroll
            for (int j = 0; j < JR; ++j) x[j] = *reinterpret_cast<const uint4 *>(verify_stage[row_slot(g * JR + j)]);
#pragma unroll
            for (int j = 0; j < JR; ++j)
              store_b128_settled<kPolicyNT>(__builtin_bit_cast(gdn_u32x4, x[j]), r, c_voff(g * JR + j),
                                            c_soff(rb, g * JR + j));
            wave_lds_sync();
          }
        } else {
#pragma unroll
          for (int j = 0; j < J; ++j) {
            const int vo = (4 * j + ls) * E < K ? lane_off + j * 64 : kOutOfRange;
            store_b128_settled<0>(__builtin_bit_cast(gdn_u32x4, pack16<S>(h[j])), r, vo, rb * 16 * row_bytes);
          }
        }
      };
      apply(0, seg);
      if (pstore_b) store(rbnd);
      apply(seg, pn);
      store(rfin);
      // The window is verified from the folded tile as stored.
#pragma unroll
      for (int j = 0; j < J; ++j) buf[j] = pack16<S>(h[j]);
    }
  };

  if (a.l2norm) {
    // kernels.py:645-648: x * rsqrt(sum(x*x) + 1e-6) for q and k, then q *= scale.
    if (lane < NV) {
      float ss = 0.0f;
      for (int kk = 0; kk < KP; ++kk) ss += m_lds[lane][kk] * m_lds[lane][kk];
      inv_lds[lane] = rsqrtf(ss + 1e-6f);
    }
    wave_lds_sync();
#pragma unroll
    for (int p = 0; p < STAGE_PASSES; ++p) {
      const int idx = p * kVerifyThreads + lane;
      const int vid = idx / C4, kk = (idx - vid * C4) * 4;
      if (vid < NV) {
        const bool is_q = vid >= QM;
        const int t = is_q ? vid - QM : vid;
        const bool wr = !is_q && key_writer && ((valid_mask >> t) & 1u) && kk < K;
        const int64_t base = int64_t(b) * a.key_rs + int64_t(key_head) * a.key_hs + int64_t(t) * a.key_ts + kk;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float x = m_lds[vid][kk + e] * inv_lds[vid];
          m_lds[vid][kk + e] = x * (is_q ? a.scale : 1.0f);
          if (wr) st_f32_or<A>(a.key, base + e, key_f32, x);
        }
      }
    }
    wave_lds_sync();
  }

  // ---- 5. Gram matrix k_s . m_j (8 lanes per dot product, DPP sum) ----
  {
    const int j8 = lane & 7;
    for (int d0 = 0; d0 < QM * NV; d0 += kVerifyThreads / 8) {
      const int d = d0 + (lane >> 3);
      const int s = d / NV, j = d - (d / NV) * NV;
      float part = 0.0f;
      if (d < QM * NV) {
        constexpr int GL = KP / 8;
#pragma unroll
        for (int e = 0; e < GL; ++e) part += m_lds[s][j8 * GL + e] * m_lds[j][j8 * GL + e];
      }
      part = dpp_sum8(part);
      if (d < QM * NV && j8 == 0) gram_lds[s][j] = part;
    }
  }
  // B operands come from LDS per chunk group inside every block: keeping all of
  // them in registers would cost the occupancy the load pipeline needs. Lanes
  // of columns >= NV read some valid row: those columns of D are never used.
  const bool col_live = li < NV;
  const int brow = li & (NV - 1);

  // ---- 6. pipelined S_0 . [k, q~] on the matrix cores, recurrence per half ----
  auto gemv_block = [&](int rb, const uint4 (&src)[J]) {
    asm volatile("" ::: "memory");  // re-read the B operands for every block
    f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < J; ++j) {
      float bop[E];
#pragma unroll
      for (int e = 0; e < E; ++e) bop[e] = m_lds[brow][E * (4 * j + ls) + e];
#pragma unroll
      for (int e = 0; e < E; ++e)
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(chunk_elem<S>(src[j], e), bop[e], acc, 0, 0, 0);
    }
    if (col_live) {
      const int rr = (rb & 3) * 16 + 4 * ls;
#pragma unroll
      for (int r = 0; r < 4; ++r) d_lds[rr + r][li] = acc[r];
    }
  };
  // Outputs and corrections go out through buffer stores that are issued for
  // every token and lane (an invalid one gets an out-of-range offset and is
  // dropped): a store skipped on some path would make the wait counts of the
  // loads still in flight assume it, and drain the pipeline at the next block.
  const bool out_f32 = a.out_f32 != 0;
  const __amdgpu_buffer_rsrc_t rout = make_rsrc(a.out, (bos * a.out_ts + out_base) * (out_f32 ? 4 : AS));
  const __amdgpu_buffer_rsrc_t rcorr =
      make_rsrc(a.corr, (int64_t(b) * a.corr_rs + int64_t(hv) * a.corr_hs + row0) * 4);
  float res_c[2][QM], res_o[2][QM];  // corrections and outputs of the lane's row in each half
  auto emit = [&](int half) {
    const int lrow = half * 64 + lane;
    int row_ok = row0 + lrow < V;
    asm volatile("" : "+v"(row_ok));  // per-lane offsets below, not branches
#pragma unroll
    for (int t = 0; t < QM; ++t) {
      const bool st = ((valid_mask >> t) & 1u) && row_ok;
      const int oel = t * int(a.out_ts) + lrow;
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(res_o[half][t]), rout,
                                            st && out_f32 ? oel * 4 : kOutOfRange, 0, 0);
      if constexpr (sizeof(A) == 2)
        __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, from_f32<A>(res_o[half][t])), rout,
                                              st && !out_f32 ? oel * AS : kOutOfRange, 0, 0);
      __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(res_c[half][t]), rcorr,
                                            st && rec_ok ? (t * a.corr_ts + lrow) * 4 : kOutOfRange, 0, 0);
    }
  };
  auto recurrence = [&](int half) {
    wave_lds_sync();  // d_lds (and, on the first half, gram_lds) complete
    float u[QM], wq[QM];
#pragma unroll
    for (int t = 0; t < QM; ++t) {
      u[t] = d_lds[lane][t];
      wq[t] = d_lds[lane][QM + t];
    }
#pragma unroll
    for (int t = 0; t < QM; ++t) {
      const bool tv = (valid_mask >> t) & 1u;
      const float d = dec[t];
      const float c = tv ? (vv[half][t] - d * u[t]) * bet[t] : 0.0f;
      if (tv) {
#pragma unroll
        for (int j = t + 1; j < QM; ++j) u[j] = __builtin_fmaf(c, gram_lds[t][j], d * u[j]);
#pragma unroll
        for (int j = t; j < QM; ++j) wq[j] = __builtin_fmaf(c, gram_lds[t][QM + j], d * wq[j]);
      }
      res_c[half][t] = c;
      res_o[half][t] = wq[t];
    }
    emit(half);
    wave_lds_sync();  // d_lds may be overwritten by the next half
  };
#pragma unroll
  for (int rb = 0; rb < NRB; rb += 2) {
    if constexpr (NT && !DEFER) {
      // Once a block sits in LDS its registers take the block after next:
      // those loads issue before the block's last read-back and its matrix
      // work.
      uint4 op[J];
      auto stage_block = [&](int next, uint4 (&buf)[J], float (&pc)[QM]) {
#pragma unroll
        for (int g = 0; g < ROUNDS; ++g) {
          stage_write(buf, g);
          if (g + 1 == ROUNDS && next < NRB) load_block(next, buf, pc);
          wave_lds_sync();
          stage_read(op, g);
          wave_lds_sync();
        }
      };
      stage_block(rb + 2, bufA, pcA);
      gemv_block(rb, op);
      stage_block(rb + 3, bufB, pcB);
      gemv_block(rb + 1, op);
    } else {
      transpose(bufA);
      fold_block(rb, bufA, pcA);
      gemv_block(rb, bufA);
      if (rb + 2 < NRB) load_block(rb + 2, bufA, pcA);
      transpose(bufB);
      fold_block(rb + 1, bufB, pcB);
      gemv_block(rb + 1, bufB);
      if (rb + 3 < NRB) load_block(rb + 3, bufB, pcB);
    }
    if (NRB == 8 && rb + 2 == NRB / 2) load_v(1);  // a half tile has no second half
    // Every half runs its recurrence, also one past V (its rows store nothing):
    // skipping it would be a path without its stores.
    if ((rb + 2) % 4 == 0) recurrence((rb + 2) / 4 - 1);
  }
}

// Rows b < a.nt_rows read their state tiles with non-temporal loads, the
// rest with ordinary ones. A launch streams its tiles once; what an ordinary
// load leaves in the memory-side cache is what a commit reading the same pages
// right after finds there, and only the last-read part of a large batch can
// still be there. Reading the earlier part non-temporally keeps it from
// evicting that part (and the non-temporal reads run faster): the host sets
// nt_rows so that the ordinary reads cover the last `retain` bytes.
template <typename S, typename A, int J, int QM, bool DEFER>
__global__ __launch_bounds__(kVerifyThreads) void verify_kernel(VerifyArgs a) {
  __shared__ VerifyLds<QM, 4 * Chunk<S>::E * J, J, DEFER> lds;
  if (DEFER || int(blockIdx.y) < a.nt_rows)  // the deferred verify: every row (see verify.hip)
    verify_wave<S, A, J, QM, DEFER, true>(a, lds);
  else
    verify_wave<S, A, J, QM, DEFER, false>(a, lds);
}

// Launch for one state type; defined per state type in verify_<state>.hip.
template <typename S>
void launch_verify_state(int act_dt, int j, int qm, bool deferred, dim3 grid, hipStream_t s, const VerifyArgs &a);

template <typename S, typename A, int J, bool DEFER>
static void launch_verify_q(int qm, dim3 grid, hipStream_t s, const VerifyArgs &a) {
  // The staging block only for launches with non-temporal rows (it costs
  // occupancy otherwise).
  const unsigned lds = DEFER || a.nt_rows > 0 ? unsigned(verify_stage_bytes(J)) : 0u;
  switch (qm) {
    case 1: hipLaunchKernelGGL((verify_kernel<S, A, J, 1, DEFER>), grid, dim3(kVerifyThreads), lds, s, a); break;
    case 2: hipLaunchKernelGGL((verify_kernel<S, A, J, 2, DEFER>), grid, dim3(kVerifyThreads), lds, s, a); break;
    case 4: hipLaunchKernelGGL((verify_kernel<S, A, J, 4, DEFER>), grid, dim3(kVerifyThreads), lds, s, a); break;
    default: hipLaunchKernelGGL((verify_kernel<S, A, J, 8, DEFER>), grid, dim3(kVerifyThreads), lds, s, a); break;
  }
}

// J: 16-byte chunks per lane per row, KP = 4 * E * J <= 256, so J <= 16 for
// f32 state and J <= 8 for 16-bit state.
template <typename S, typename A, bool DEFER>
static void launch_verify_j(int j, int qm, dim3 grid, hipStream_t s, const VerifyArgs &a) {
  switch (j) {
    case 1: launch_verify_q<S, A, 1, DEFER>(qm, grid, s, a); break;
    case 2: launch_verify_q<S, A, 2, DEFER>(qm, grid, s, a); break;
    case 4: launch_verify_q<S, A, 4, DEFER>(qm, grid, s, a); break;
    case 8: launch_verify_q<S, A, 8, DEFER>(qm, grid, s, a); break;
    default:
      if constexpr (Chunk<S>::E == 4) launch_verify_q<S, A, 16, DEFER>(qm, grid, s, a);
      break;
  }
}

template <typename S, bool DEFER>
static void launch_verify_act(int act_dt, int j, int qm, dim3 grid, hipStream_t s, const VerifyArgs &a) {
  switch (act_dt) {
    case GDN_DT_BF16: launch_verify_j<S, bf16, DEFER>(j, qm, grid, s, a); break;
    case GDN_DT_F16: launch_verify_j<S, f16, DEFER>(j, qm, grid, s, a); break;
    default: launch_verify_j<S, float, DEFER>(j, qm, grid, s, a); break;
  }
}

// The deferred-commit kernels of each state type live in a translation unit of
// their own (verify_<state>_deferred.hip), so the halves compile in parallel.
template <typename S>
void launch_verify_deferred(int act_dt, int j, int qm, dim3 grid, hipStream_t s, const VerifyArgs &a);

#define GDN_DEFINE_VERIFY_LAUNCH(STATE)                                                                \
  template <>                                                                                          \
  void launch_verify_state<STATE>(int act_dt, int j, int qm, bool deferred, dim3 grid, hipStream_t s, \
                                  const VerifyArgs &a) {                                               \
    if (deferred)                                                                                      \
      launch_verify_deferred<STATE>(act_dt, j, qm, grid, s, a);                                        \
    else                                                                                               \
      launch_verify_act<STATE, false>(act_dt, j, qm, grid, s, a);                                      \
  }

#define GDN_DEFINE_VERIFY_DEFERRED_LAUNCH(STATE)                                                         \
  template <>                                                                                            \
  void launch_verify_deferred<STATE>(int act_dt, int j, int qm, dim3 grid, hipStream_t s,                \
                                     const VerifyArgs &a) {                                              \
    launch_verify_act<STATE, true>(act_dt, j, qm, grid, s, a);                                           \
  }

}  // namespace gdn
