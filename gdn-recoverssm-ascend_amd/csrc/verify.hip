// Speculative verify of a Gated DeltaNet window from the read-only checkpoint
// (kernels.py:491-697 and csrc/verify.h:284-332 of the reference plugin).
//
// Per (row b, value head hv) the reference advances S <- S*d_t + c_t k_t^T
// token by token. Because verify never writes the state back, this kernel never
// forms S_t: with G_t = d_0 ... d_t,
//     S_{t-1} k_t = G_{t-1} S_0 k_t + sum_{s<t} (G_{t-1}/G_s) (k_s.k_t) c_s
//     S_t q~_t    = G_t     S_0 q~_t + sum_{s<=t} (G_t/G_s)   (k_s.q~_t) c_s
// so the state is needed only through the 2Q matrix-vector products
// S_0 [k_0 .. k_{Q-1}, q~_0 .. q~_{Q-1}] (2Q FMAs per state element, read once
// from HBM), and the per-row recurrence runs on Q-vectors with the tiny Gram
// matrix k_s.{k_t, q~_t}; it is evaluated incrementally (no divisions):
//     u_j <- d_t u_j + c_t (k_t.k_j),  w_j <- d_t w_j + c_t (k_t.q~_j).
//
// Work decomposition: one workgroup (4 waves) per (row, value head, 128-row
// tile of V). Lane l of wave w owns rows w*32 + (l>>3) + 8i (i = 0..3) and the
// 16-byte chunks (l&7) + 8c of each of them, so every wave load instruction
// covers eight full 128-byte lines. Dot products are summed over the 8 lanes of
// a row group with DPP; the k/q vectors, the Gram matrix and v are staged in LDS.
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
  int64_t rows, tokens, heads, value_heads, Q, blocks, record_rows, null_block;
  int64_t q_ts, k_ts, v_ts, g_ts, beta_ts;
  int64_t state_bs, state_hs, state_vs;
  int64_t corr_rs, corr_hs, corr_ts;
  int64_t key_rs, key_hs, key_ts;
  int64_t decay_rs, decay_hs, decay_ts;
  int64_t out_ts, qsl_s, idx_s;
  float scale;
  int32_t K, V, KP, NVT;
  int32_t act_dt, out_dt, beta_dt, g_dt, key_dt, qsl_dt, idx_dt;
  int32_t l2norm, key_per_value_head;
};

constexpr int kVerifyThreads = 256;
constexpr int kTileRows = 128;  // rows of V per workgroup: 4 waves x 32 rows

template <typename S, int CPL, int QM>
__global__ __launch_bounds__(kVerifyThreads) void verify_kernel(VerifyArgs a) {
  constexpr int E = Chunk<S>::E;
  constexpr int KP = 8 * CPL * E;  // padded K covered by the 8 lanes of a row group
  constexpr int NV = 2 * QM;       // vectors: k_0..k_{QM-1}, q~_0..q~_{QM-1}
  __shared__ float m_lds[NV][KP];
  __shared__ float gram_lds[QM][NV];
  __shared__ float v_lds[QM][kTileRows];

  const int64_t w_id = blockIdx.x;
  const int vt = int(w_id % a.NVT);
  const int64_t hv = (w_id / a.NVT) % a.value_heads;
  const int64_t b = w_id / (int64_t(a.NVT) * a.value_heads);
  const int64_t ratio = a.value_heads / a.heads;
  const int64_t h = hv / ratio;
  const int tid = threadIdx.x;
  const int V = a.V;
  const int row0 = vt * kTileRows;

  const int64_t bos = load_index(a.qsl, b * a.qsl_s, a.qsl_dt);
  const int64_t eos = load_index(a.qsl, (b + 1) * a.qsl_s, a.qsl_dt);
  const int64_t qlen = eos - bos;
  const int64_t slot = load_index(a.indices, b * a.idx_s, a.idx_dt);
  const int Q = int(a.Q);

  if (slot <= a.null_block || slot >= a.blocks) {
    // Null or out-of-range page: zero outputs for the window, records untouched
    // (kernels.py:569-583).
    for (int t = 0; t < Q; ++t) {
      const int64_t tok = bos + t;
      if (!(t < qlen && tok >= 0 && tok < a.tokens)) continue;
      for (int r = tid; r < kTileRows; r += kVerifyThreads) {
        const int vr = row0 + r;
        if (vr < V) store_from_f32(a.out, tok * a.out_ts + hv * V + vr, a.out_dt, 0.0f);
      }
    }
    return;
  }
  // Token validity is uniform across the workgroup (kernels.py:612).
  uint32_t valid_mask = 0;
  for (int t = 0; t < QM; ++t) {
    const int64_t tok = bos + t;
    if (t < Q && t < qlen && tok >= 0 && tok < a.tokens) valid_mask |= 1u << t;
  }
  if (valid_mask == 0) return;

  // ---- 1. issue the state loads (the only large HBM read) ----
  const int wave = tid >> 6, lane = tid & 63;
  const int grp = lane >> 3, j8 = lane & 7;
  const S *sp = static_cast<const S *>(a.state) + slot * a.state_bs + hv * a.state_hs;
  uint4 raw[4][CPL];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int vr = row0 + wave * 32 + grp + 8 * i;
#pragma unroll
    for (int c = 0; c < CPL; ++c) {
      const int kc = j8 + 8 * c;
      raw[i][c] = (vr < V && kc * E < a.K) ? *reinterpret_cast<const uint4 *>(sp + vr * a.state_vs + kc * E)
                                           : make_uint4(0, 0, 0, 0);
    }
  }

  // ---- 2. stage k_t, q~_t (fp32, zero padded) and v; write key/decay records ----
  const bool rec_ok = b < a.record_rows;
  const bool key_writer = rec_ok && vt == 0 && (a.key_per_value_head || (hv % ratio) == 0);
  const int64_t key_head = a.key_per_value_head ? hv : h;
  constexpr int SL = KP / 32;  // elements per thread when 32 threads stage one vector
  for (int vid0 = 0; vid0 < NV; vid0 += kVerifyThreads / 32) {
    const int vid = vid0 + (tid >> 5);
    const int sub = tid & 31;
    if (vid < NV) {
      const bool is_q = vid >= QM;
      const int t = is_q ? vid - QM : vid;
      const bool tv = (valid_mask >> t) & 1u;
      const int64_t tok = bos + t;
      float x[SL];
      float ss = 0.0f;
#pragma unroll
      for (int e = 0; e < SL; ++e) {
        const int kk = sub * SL + e;
        x[e] = (tv && kk < a.K) ? load_as_f32(is_q ? a.q : a.k, tok * (is_q ? a.q_ts : a.k_ts) + h * a.K + kk, a.act_dt)
                                : 0.0f;
        ss += x[e] * x[e];
      }
      float key_val[SL];
#pragma unroll
      for (int e = 0; e < SL; ++e) key_val[e] = x[e];
      if (a.l2norm) {
        // kernels.py:645-648: x * rsqrt(sum(x*x) + 1e-6), the sum over the 32
        // threads staging this vector.
#pragma unroll
        for (int off = 16; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 32);
        const float inv = rsqrtf(ss + 1e-6f);
#pragma unroll
        for (int e = 0; e < SL; ++e) {
          x[e] *= inv;
          key_val[e] = x[e];
        }
      }
      if (is_q) {
#pragma unroll
        for (int e = 0; e < SL; ++e) x[e] *= a.scale;
      }
#pragma unroll
      for (int e = 0; e < SL; ++e) m_lds[vid][sub * SL + e] = x[e];
      if (!is_q && tv && key_writer) {
#pragma unroll
        for (int e = 0; e < SL; ++e) {
          const int kk = sub * SL + e;
          if (kk < a.K) store_from_f32(a.key, b * a.key_rs + key_head * a.key_hs + t * a.key_ts + kk, a.key_dt, key_val[e]);
        }
      }
    }
  }
  for (int idx = tid; idx < QM * kTileRows; idx += kVerifyThreads) {
    const int t = idx / kTileRows, r = idx % kTileRows;
    const int vr = row0 + r;
    const bool tv = (valid_mask >> t) & 1u;
    v_lds[t][r] = (tv && vr < V) ? load_as_f32(a.v, (bos + t) * a.v_ts + hv * V + vr, a.act_dt) : 0.0f;
  }
  float dec[QM], bet[QM];
#pragma unroll
  for (int t = 0; t < QM; ++t) {
    const bool tv = (valid_mask >> t) & 1u;
    const int64_t tok = bos + t;
    dec[t] = tv ? expf(load_as_f32(a.g, tok * a.g_ts + hv, a.g_dt)) : 1.0f;
    bet[t] = tv ? load_as_f32(a.beta, tok * a.beta_ts + hv, a.beta_dt) : 0.0f;
  }
  if (rec_ok && vt == 0 && tid < QM && ((valid_mask >> tid) & 1u))
    a.decay[b * a.decay_rs + hv * a.decay_hs + tid * a.decay_ts] =
        expf(load_as_f32(a.g, (bos + tid) * a.g_ts + hv, a.g_dt));
  __syncthreads();

  // ---- 3. Gram matrix k_s . m_j (8 lanes per dot product) ----
  for (int d0 = 0; d0 < QM * NV; d0 += kVerifyThreads / 8) {
    const int d = d0 + (tid >> 3);
    float part = 0.0f;
    const int s = d / NV, j = d % NV;
    if (d < QM * NV) {
      constexpr int GL = KP / 8;
#pragma unroll
      for (int e = 0; e < GL; ++e) part += m_lds[s][j8 * GL + e] * m_lds[j][j8 * GL + e];
    }
    part = dpp_sum8(part);
    if (d < QM * NV && j8 == 0) gram_lds[s][j] = part;
  }

  // ---- 4. S_0 . m_j for the lane's 4 rows ----
  float sv[4][CPL][E];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int c = 0; c < CPL; ++c) unpack16<S>(raw[i][c], sv[i][c]);
  float p[4][NV];
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    const int t = j < QM ? j : j - QM;
    if (t < Q) {
      float m[CPL][E];
#pragma unroll
      for (int c = 0; c < CPL; ++c)
#pragma unroll
        for (int e = 0; e < E; ++e) m[c][e] = m_lds[j][(j8 + 8 * c) * E + e];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float acc = 0.0f;
#pragma unroll
        for (int c = 0; c < CPL; ++c)
#pragma unroll
          for (int e = 0; e < E; ++e) acc = __builtin_fmaf(sv[i][c][e], m[c][e], acc);
        p[i][j] = acc;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) p[i][j] = 0.0f;
    }
  }
#pragma unroll
  for (int j = 0; j < NV; ++j) {
    if ((j < QM ? j : j - QM) < Q) {
#pragma unroll
      for (int i = 0; i < 4; ++i) p[i][j] = dpp_sum8(p[i][j]);
    }
  }
  __syncthreads();  // Gram visible

  // ---- 5. per-row recurrence: lanes 2i, 2i+1 of a row group own row i ----
  const int isel = j8 >> 1;
  float u[QM], wq[QM];
  const bool sel_odd = (isel & 1) != 0, sel_hi = (isel & 2) != 0;
#pragma unroll
  for (int t = 0; t < QM; ++t) {
    float x0 = p[0][t], x1 = p[1][t], x2 = p[2][t], x3 = p[3][t];
    float y0 = p[0][QM + t], y1 = p[1][QM + t], y2 = p[2][QM + t], y3 = p[3][QM + t];
    // Keep the per-lane choice a register select: without the barrier the
    // compiler turns it into a select of addresses into `p`, which then can no
    // longer live in registers.
    asm volatile("" : "+v"(x0), "+v"(x1), "+v"(x2), "+v"(x3));
    asm volatile("" : "+v"(y0), "+v"(y1), "+v"(y2), "+v"(y3));
    u[t] = sel_odd ? (sel_hi ? x3 : x1) : (sel_hi ? x2 : x0);
    wq[t] = sel_odd ? (sel_hi ? y3 : y1) : (sel_hi ? y2 : y0);
  }
  const int lrow = wave * 32 + grp + 8 * isel;
  const int vr = row0 + lrow;
  const bool row_ok = vr < V;
  const bool writes_out = (j8 & 1) != 0;
  float *corr_row = a.corr + b * a.corr_rs + hv * a.corr_hs + vr;
#pragma unroll
  for (int t = 0; t < QM; ++t) {
    if ((valid_mask >> t) & 1u) {
      const float d = dec[t];
      const float skt = d * u[t];
      const float c = (v_lds[t][lrow] - skt) * bet[t];
#pragma unroll
      for (int j = t + 1; j < QM; ++j) u[j] = __builtin_fmaf(c, gram_lds[t][j], d * u[j]);
#pragma unroll
      for (int j = t; j < QM; ++j) wq[j] = __builtin_fmaf(c, gram_lds[t][QM + j], d * wq[j]);
      if (row_ok) {
        if (writes_out)
          store_from_f32(a.out, (bos + t) * a.out_ts + hv * V + vr, a.out_dt, wq[t]);
        else if (rec_ok)
          corr_row[t * a.corr_ts] = c;
      }
    }
  }
}

template <typename S, int CPL>
static void launch_verify_q(int qm, dim3 grid, hipStream_t s, const VerifyArgs &a) {
  switch (qm) {
    case 1: hipLaunchKernelGGL((verify_kernel<S, CPL, 1>), grid, dim3(kVerifyThreads), 0, s, a); break;
    case 2: hipLaunchKernelGGL((verify_kernel<S, CPL, 2>), grid, dim3(kVerifyThreads), 0, s, a); break;
    case 4: hipLaunchKernelGGL((verify_kernel<S, CPL, 4>), grid, dim3(kVerifyThreads), 0, s, a); break;
    default: hipLaunchKernelGGL((verify_kernel<S, CPL, 8>), grid, dim3(kVerifyThreads), 0, s, a); break;
  }
}

// Chunks per lane per row: KP = 8 * CPL * E <= 256, so CPL <= 8 for f32 state
// and CPL <= 4 for 16-bit state.
template <typename S>
static void launch_verify_k(int cpl, int qm, dim3 grid, hipStream_t s, const VerifyArgs &a) {
  switch (cpl) {
    case 1: launch_verify_q<S, 1>(qm, grid, s, a); break;
    case 2: launch_verify_q<S, 2>(qm, grid, s, a); break;
    case 4: launch_verify_q<S, 4>(qm, grid, s, a); break;
    default:
      if constexpr (Chunk<S>::E == 4) launch_verify_q<S, 8>(qm, grid, s, a);
      break;
  }
}

static bool act_dtype_ok(int32_t dt) { return dt == GDN_DT_F32 || dt == GDN_DT_BF16 || dt == GDN_DT_F16; }

}  // namespace gdn

using namespace gdn;

extern "C" int gdn_recoverssm_verify(const void *q, const void *k, const void *v, const void *g, const void *beta,
                                     const void *state, void *correction, void *key, void *decay, void *out,
                                     const void *qsl, const void *indices, const int64_t *config,
                                     int64_t config_len, float scale, const gdn_verify_ext *ext, void *stream) {
  if (!config || config_len != GDN_VERIFY_CONFIG_FIELDS || !ext) {
    set_error("verify: tiling ABI expects %d config fields and an extension block", GDN_VERIFY_CONFIG_FIELDS);
    return GDN_ERR_INVALID;
  }
  // Field order of the reference's GDN_VERIFY_FIELDS (csrc/common.h:8-36).
  VerifyArgs a{};
  a.rows = config[0];
  a.tokens = config[1];
  a.heads = config[2];
  a.value_heads = config[3];
  a.Q = config[4];
  a.blocks = config[5];
  a.record_rows = config[6];
  a.null_block = config[7];
  a.q_ts = config[8];
  a.k_ts = config[9];
  a.v_ts = config[10];
  a.g_ts = config[11];
  a.beta_ts = config[12];
  a.state_bs = config[13];
  a.state_hs = config[14];
  a.state_vs = config[15];
  a.corr_rs = config[16];
  a.corr_hs = config[17];
  a.corr_ts = config[18];
  a.key_rs = config[19];
  a.key_hs = config[20];
  a.key_ts = config[21];
  a.decay_rs = config[22];
  a.decay_hs = config[23];
  a.decay_ts = config[24];
  a.out_ts = config[25];
  a.qsl_s = config[26];
  a.idx_s = config[27];
  a.scale = scale;
  if (a.rows < 0 || a.tokens < 0 || a.heads <= 0 || a.value_heads <= 0 || a.value_heads % a.heads != 0 ||
      a.Q < 1 || a.Q > 8 || a.blocks <= 0 || a.record_rows < 0 || a.tokens > a.rows * a.Q) {
    set_error("verify: geometry rows=%lld tokens=%lld heads=%lld value_heads=%lld Q=%lld", (long long)a.rows,
              (long long)a.tokens, (long long)a.heads, (long long)a.value_heads, (long long)a.Q);
    return GDN_ERR_INVALID;
  }
  if (!act_dtype_ok(ext->act_dtype) || !act_dtype_ok(ext->out_dtype) || !act_dtype_ok(ext->state_dtype) || !act_dtype_ok(ext->key_record_dtype) ||
      !act_dtype_ok(ext->beta_dtype) || !act_dtype_ok(ext->g_dtype) ||
      (ext->qsl_dtype != GDN_DT_I32 && ext->qsl_dtype != GDN_DT_I64) ||
      (ext->index_dtype != GDN_DT_I32 && ext->index_dtype != GDN_DT_I64)) {
    set_error("verify: unsupported dtype combination");
    return GDN_ERR_UNSUPPORTED;
  }
  const int E = ext->state_dtype == GDN_DT_F32 ? 4 : 8;
  const int64_t K = ext->key_dim, V = ext->value_dim;
  if (K < 1 || K > 256 || K % E != 0 || V < 1 || a.state_vs % E != 0 || a.state_hs % E != 0 ||
      a.state_bs % E != 0 || (reinterpret_cast<uintptr_t>(state) & 15u) != 0) {
    set_error("verify: state layout K=%lld V=%lld unsupported (K <= 256, multiple of %d, 16-byte aligned rows)",
              (long long)K, (long long)V, E);
    return GDN_ERR_UNSUPPORTED;
  }
  if (a.rows == 0 || a.tokens == 0) return GDN_OK;
  if (!q || !k || !v || !g || !beta || !state || !correction || !key || !decay || !out || !qsl || !indices) {
    set_error("verify: null tensor pointer");
    return GDN_ERR_INVALID;
  }
  a.q = q;
  a.k = k;
  a.v = v;
  a.g = g;
  a.beta = beta;
  a.state = state;
  a.corr = static_cast<float *>(correction);
  a.key = key;
  a.decay = static_cast<float *>(decay);
  a.out = out;
  a.qsl = qsl;
  a.indices = indices;
  a.K = int32_t(K);
  a.V = int32_t(V);
  a.act_dt = ext->act_dtype;
  a.out_dt = ext->out_dtype;
  a.beta_dt = ext->beta_dtype;
  a.g_dt = ext->g_dtype;
  a.key_dt = ext->key_record_dtype;
  a.qsl_dt = ext->qsl_dtype;
  a.idx_dt = ext->index_dtype;
  a.l2norm = ext->qk_l2norm;
  a.key_per_value_head = ext->key_per_value_head;
  int cpl = 1;
  while (8 * cpl * E < K) cpl *= 2;
  const int qm = a.Q <= 1 ? 1 : a.Q <= 2 ? 2 : a.Q <= 4 ? 4 : 8;
  a.KP = 8 * cpl * E;
  a.NVT = int32_t((V + kTileRows - 1) / kTileRows);
  const int64_t grid = a.rows * a.value_heads * a.NVT;
  if (grid > 0x7fffffffLL) {
    set_error("verify: grid too large");
    return GDN_ERR_UNSUPPORTED;
  }
  auto s = static_cast<hipStream_t>(stream);
  const dim3 gd(static_cast<unsigned>(grid), 1u, 1u);
  switch (ext->state_dtype) {
    case GDN_DT_BF16: launch_verify_k<bf16>(cpl, qm, gd, s, a); break;
    case GDN_DT_F16: launch_verify_k<f16>(cpl, qm, gd, s, a); break;
    default: launch_verify_k<float>(cpl, qm, gd, s, a); break;
  }
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error("verify: launch failed: %s", hipGetErrorString(err));
    return GDN_ERR_LAUNCH;
  }
  return GDN_OK;
}
