// C entry point of the verify kernel: argument validation and dispatch over
// the state / activation types (kernels in verify_kernel.cuh, instantiated in
// verify_{f32,bf16,f16}.hip).
#include "verify_kernel.cuh"

namespace gdn {

static bool float_dt_ok(int32_t dt) { return dt == GDN_DT_F32 || dt == GDN_DT_BF16 || dt == GDN_DT_F16; }

static bool fits_i32(int64_t x) { return x >= INT32_MIN && x <= INT32_MAX; }

}  // namespace gdn

using namespace gdn;

static int verify_impl(const void *q, const void *k, const void *v, const void *g, const void *beta,
                       const void *state, void *correction, void *key, void *decay, void *out, const void *qsl,
                       const void *indices, const int64_t *config, int64_t config_len, float scale,
                       const gdn_verify_ext *ext, const void *a_log, const void *dt_bias,
                       const gdn_gating_ext *gating, const gdn_pending_commit *pending, void *stream) {
  if (!config || config_len != GDN_VERIFY_CONFIG_FIELDS || !ext) {
    set_error("verify: tiling ABI expects %d config fields and an extension block", GDN_VERIFY_CONFIG_FIELDS);
    return GDN_ERR_INVALID;
  }
  // Field order of the reference's GDN_VERIFY_FIELDS (csrc/common.h:8-36).
  const int64_t rows = config[0], tokens = config[1], heads = config[2], value_heads = config[3];
  const int64_t Q = config[4], blocks = config[5], record_rows = config[6], null_block = config[7];
  if (rows < 0 || tokens < 0 || heads <= 0 || value_heads <= 0 || value_heads % heads != 0 || Q < 1 || Q > 8 ||
      blocks <= 0 || record_rows < 0 || tokens > rows * Q) {
    set_error("verify: geometry rows=%lld tokens=%lld heads=%lld value_heads=%lld Q=%lld", (long long)rows,
              (long long)tokens, (long long)heads, (long long)value_heads, (long long)Q);
    return GDN_ERR_INVALID;
  }
  const int32_t act = ext->act_dtype;
  auto act_or_f32 = [act](int32_t dt) { return dt == act || dt == GDN_DT_F32; };
  if (!float_dt_ok(act) || !float_dt_ok(ext->state_dtype) || !act_or_f32(ext->out_dtype) ||
      !act_or_f32(ext->key_record_dtype) || !act_or_f32(ext->beta_dtype) || !act_or_f32(ext->g_dtype) ||
      (ext->qsl_dtype != GDN_DT_I32 && ext->qsl_dtype != GDN_DT_I64) ||
      (ext->index_dtype != GDN_DT_I32 && ext->index_dtype != GDN_DT_I64)) {
    set_error("verify: unsupported dtype combination (out, key record, gate and beta must be FP32 or the "
              "activation dtype)");
    return GDN_ERR_UNSUPPORTED;
  }
  const int E = ext->state_dtype == GDN_DT_F32 ? 4 : 8;
  const int64_t K = ext->key_dim, V = ext->value_dim;
  const int64_t state_bs = config[13], state_hs = config[14], state_vs = config[15];
  if (K < 1 || K > 256 || K % E != 0 || V < 1 || state_vs % E != 0 || state_hs % E != 0 || state_bs % E != 0 ||
      !fits_i32(state_hs) || !fits_i32(state_vs * V) || state_vs * (ext->state_dtype == GDN_DT_F32 ? 4 : 2) >= (1 << 24) ||
      (reinterpret_cast<uintptr_t>(state) & 15u) != 0) {
    set_error("verify: state layout K=%lld V=%lld unsupported (K <= 256, multiple of %d, 16-byte aligned rows)",
              (long long)K, (long long)V, E);
    return GDN_ERR_UNSUPPORTED;
  }
  if (rows > 65535) {
    set_error("verify: %lld rows exceed the 65535-row grid", (long long)rows);
    return GDN_ERR_UNSUPPORTED;
  }
  // Every stride and count the kernel takes in 32 bits.
  for (int i : {5, 7, 8, 9, 10, 11, 12, 13, 16, 17, 18, 19, 20, 21, 22, 23, 24, 25, 26, 27}) {
    if (!fits_i32(config[i])) {
      set_error("verify: config field %d (%lld) exceeds 32 bits", i, (long long)config[i]);
      return GDN_ERR_UNSUPPORTED;
    }
  }
  // Activations are read through 32-bit offsets from each row's first token.
  const int64_t act_b = act == GDN_DT_F32 ? 4 : 2;
  auto window_ok = [Q](int64_t ts, int64_t width, int64_t esz) {
    return ts >= 0 && ((Q - 1) * ts + width) * esz + 16 < int64_t(kWindowBytes);
  };
  if (!window_ok(config[8], heads * K, act_b) || !window_ok(config[9], heads * K, act_b) ||
      !window_ok(config[10], value_heads * V, act_b) || !window_ok(config[11], value_heads, 4) ||
      !window_ok(config[12], value_heads, 4) ||
      !window_ok(config[25], value_heads * V, ext->out_dtype == GDN_DT_F32 ? 4 : act_b) ||
      !window_ok(config[18], V, 4)) {
    set_error("verify: activation / output / correction token strides must be non-negative and span under 2 GiB "
              "per window");
    return GDN_ERR_UNSUPPORTED;
  }
  if (gating && (!float_dt_ok(gating->a_log_dtype) || !float_dt_ok(gating->dt_bias_dtype) ||
                 !(gating->softplus_beta > 0.0f))) {
    set_error("verify: gating parameters need FP32/BF16/F16 A_log and dt_bias and a positive softplus beta");
    return GDN_ERR_UNSUPPORTED;
  }
  if (pending) {
    const bool ok = pending->record_rows > 0 && pending->num_rows > 0 && pending->num_rows <= INT32_MAX &&
                    act_or_f32(pending->key_dtype) && fits_i32(pending->corr_strides[0]) &&
                    fits_i32(pending->key_strides[0]) && fits_i32(pending->decay_strides[0]) &&
                    fits_i32(pending->corr_strides[1]) &&
                    fits_i32(pending->corr_strides[2]) && fits_i32(pending->key_strides[1]) &&
                    fits_i32(pending->key_strides[2]) && fits_i32(pending->decay_strides[1]) &&
                    fits_i32(pending->decay_strides[2]) &&
                    (Q - 1) * pending->corr_strides[2] + V < int64_t(kWindowBytes) / 4 &&
                    (Q - 1) * pending->key_strides[2] + K < int64_t(kWindowBytes) / 4;
    if (!ok) {
      set_error("verify_deferred: a pending plan of at least one row, FP32 or activation-typed pending keys and "
                "32-bit record strides are required");
      return GDN_ERR_UNSUPPORTED;
    }
  }
  // With nothing to verify, only pending commits give the launch work.
  if (rows == 0 || (tokens == 0 && !pending)) return GDN_OK;
  const bool need_window = tokens > 0;
  if (!state || !qsl || !indices ||
      (need_window && (!q || !k || !v || !g || !beta || !correction || !key || !decay || !out)) ||
      (gating && (!a_log || !dt_bias))) {
    set_error("verify: null tensor pointer");
    return GDN_ERR_INVALID;
  }
  VerifyArgs a{};
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
  a.tokens = int32_t(tokens);
  a.heads = int32_t(heads);
  a.value_heads = int32_t(value_heads);
  a.Q = int32_t(Q);
  a.blocks = int32_t(blocks);
  a.record_rows = int32_t(record_rows);
  a.null_block = int32_t(null_block);
  a.q_ts = int32_t(config[8]);
  a.k_ts = int32_t(config[9]);
  a.v_ts = int32_t(config[10]);
  a.g_ts = int32_t(config[11]);
  a.beta_ts = int32_t(config[12]);
  a.state_bs = int32_t(state_bs);
  a.state_hs = int32_t(state_hs);
  a.state_vs = int32_t(state_vs);
  a.corr_rs = int32_t(config[16]);
  a.corr_hs = int32_t(config[17]);
  a.corr_ts = int32_t(config[18]);
  a.key_rs = int32_t(config[19]);
  a.key_hs = int32_t(config[20]);
  a.key_ts = int32_t(config[21]);
  a.decay_rs = int32_t(config[22]);
  a.decay_hs = int32_t(config[23]);
  a.decay_ts = int32_t(config[24]);
  a.out_ts = int32_t(config[25]);
  a.qsl_s = int32_t(config[26]);
  a.idx_s = int32_t(config[27]);
  a.scale = scale;
  a.K = int32_t(K);
  a.V = int32_t(V);
  a.qsl_i64 = ext->qsl_dtype == GDN_DT_I64;
  a.idx_i64 = ext->index_dtype == GDN_DT_I64;
  a.g_f32 = ext->g_dtype == GDN_DT_F32;
  a.beta_f32 = ext->beta_dtype == GDN_DT_F32;
  a.key_f32 = ext->key_record_dtype == GDN_DT_F32;
  a.out_f32 = ext->out_dtype == GDN_DT_F32;
  a.l2norm = ext->qk_l2norm;
  a.key_per_value_head = ext->key_per_value_head;
  if (pending) {
    if (!pending->rows || !pending->source || !pending->lengths || !pending->final_indices ||
        !pending->boundary_indices || !pending->boundary_lengths || !pending->correction || !pending->key ||
        !pending->decay) {
      set_error("verify_deferred: null pending-commit pointer");
      return GDN_ERR_INVALID;
    }
    if (pending->correction == correction || pending->key == key || pending->decay == decay) {
      set_error("verify_deferred: the pending commit's records are the buffers this verify writes");
      return GDN_ERR_INVALID;
    }
    a.p_rows = pending->rows;
    a.p_src = pending->source;
    a.p_len = pending->lengths;
    a.p_final = pending->final_indices;
    a.p_bnd = pending->boundary_indices;
    a.p_blen = pending->boundary_lengths;
    a.p_corr = static_cast<const float *>(pending->correction);
    a.p_key = pending->key;
    a.p_decay = static_cast<const float *>(pending->decay);
    a.p_corr_rs = int32_t(pending->corr_strides[0]);
    a.p_corr_hs = int32_t(pending->corr_strides[1]);
    a.p_corr_ts = int32_t(pending->corr_strides[2]);
    a.p_key_rs = int32_t(pending->key_strides[0]);
    a.p_key_hs = int32_t(pending->key_strides[1]);
    a.p_key_ts = int32_t(pending->key_strides[2]);
    a.p_decay_rs = int32_t(pending->decay_strides[0]);
    a.p_decay_hs = int32_t(pending->decay_strides[1]);
    a.p_decay_ts = int32_t(pending->decay_strides[2]);
    a.p_key_f32 = pending->key_dtype == GDN_DT_F32;
    a.p_key_per_value_head = pending->key_per_value_head;
    a.p_record_rows = int32_t(pending->record_rows > 0x7fffffff ? 0x7fffffff : pending->record_rows);
    a.p_num_rows = int32_t(pending->num_rows);
  }
  if (gating) {
    a.gated = 1;
    a.a_log = a_log;
    a.dt_bias = dt_bias;
    a.a_log_dt = gating->a_log_dtype;
    a.dt_bias_dt = gating->dt_bias_dtype;
    a.softplus_beta = gating->softplus_beta;
    a.softplus_threshold = gating->softplus_threshold;
  }
  int j = 1;
  while (4 * E * j < K) j *= 2;
  const int qm = Q <= 1 ? 1 : Q <= 2 ? 2 : Q <= 4 ? 4 : 8;
  const int tile = verify_tile_rows(pending != nullptr);
  a.NVT = int32_t((V + tile - 1) / tile);
  if (int64_t(a.NVT) * value_heads > 0x7fffffffLL) {
    set_error("verify: grid too large");
    return GDN_ERR_UNSUPPORTED;
  }
  // Rows read with ordinary loads: enough of the last rows to cover the
  // retained bytes; the rows before them read their pages non-temporally.
  // The deferred verify reads and writes every row non-temporally: the
  // pages it folds are next read by the following step's verify, never
  // right after.
  if (pending) {
    a.nt_rows = int32_t(rows);
  } else {
    const int64_t row_state = value_heads * V * state_vs * (E == 4 ? 4 : 2);
    const int64_t keep = ext->state_cache_retain > 0   ? ext->state_cache_retain
                         : ext->state_cache_retain < 0 ? 0
                                                       : state_cache_retain();
    const int64_t keep_rows = row_state <= 0 ? rows : keep / row_state + (keep % row_state != 0);
    a.nt_rows = int32_t(rows > keep_rows ? rows - keep_rows : 0);
  }
  auto s = static_cast<hipStream_t>(stream);
  const dim3 gd(static_cast<unsigned>(a.NVT * value_heads), static_cast<unsigned>(rows), 1u);
  switch (ext->state_dtype) {
    case GDN_DT_BF16: launch_verify_state<bf16>(act, j, qm, pending != nullptr, gd, s, a); break;
    case GDN_DT_F16: launch_verify_state<f16>(act, j, qm, pending != nullptr, gd, s, a); break;
    default: launch_verify_state<float>(act, j, qm, pending != nullptr, gd, s, a); break;
  }
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error("verify: launch failed: %s", hipGetErrorString(err));
    return GDN_ERR_LAUNCH;
  }
  return GDN_OK;
}

extern "C" int gdn_recoverssm_verify(const void *q, const void *k, const void *v, const void *g, const void *beta,
                                     const void *state, void *correction, void *key, void *decay, void *out,
                                     const void *qsl, const void *indices, const int64_t *config,
                                     int64_t config_len, float scale, const gdn_verify_ext *ext, void *stream) {
  return verify_impl(q, k, v, g, beta, state, correction, key, decay, out, qsl, indices, config, config_len, scale,
                     ext, nullptr, nullptr, nullptr, nullptr, stream);
}

extern "C" int gdn_recoverssm_verify_deferred(const void *q, const void *k, const void *v, const void *g,
                                              const void *beta, const void *state, void *correction, void *key,
                                              void *decay, void *out, const void *qsl, const void *indices,
                                              const int64_t *config, int64_t config_len, float scale,
                                              const gdn_verify_ext *ext, const gdn_pending_commit *pending,
                                              void *stream) {
  if (!pending) {
    set_error("verify_deferred: missing pending commit");
    return GDN_ERR_INVALID;
  }
  return verify_impl(q, k, v, g, beta, state, correction, key, decay, out, qsl, indices, config, config_len, scale,
                     ext, nullptr, nullptr, nullptr, pending, stream);
}

extern "C" int gdn_recoverssm_verify_gated(const void *q, const void *k, const void *v, const void *a, const void *b,
                                           const void *a_log, const void *dt_bias, const void *state,
                                           void *correction, void *key, void *decay, void *out, const void *qsl,
                                           const void *indices, const int64_t *config, int64_t config_len,
                                           float scale, const gdn_verify_ext *ext, const gdn_gating_ext *gating,
                                           void *stream) {
  if (!gating) {
    set_error("verify_gated: missing gating parameters");
    return GDN_ERR_INVALID;
  }
  return verify_impl(q, k, v, a, b, state, correction, key, decay, out, qsl, indices, config, config_len, scale, ext,
                     a_log, dt_bias, gating, nullptr, stream);
}
