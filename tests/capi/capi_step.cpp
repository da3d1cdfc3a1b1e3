// One verify + commit step driven through the C ABI alone: hipMalloc'd
// buffers, no Python and no torch, the way a native serving runtime binds
// libgdn_recoverssm_hip.so. Test infrastructure for tests/test_gpu_capi.py,
// which writes the problem to <dir> and checks what this program writes back
// against the CPU oracle.
//
// <dir>/meta.txt holds "name value" lines (B T H HV K V Q NB W BS CD CW SCALE);
// the inputs are raw little-endian arrays: q, k, v (bf16 bits), g, beta (f32),
// state (f32 [NB, HV, V, K]), conv (bf16 bits [NB, CD, CW]), qsl, idx,
// accepted, table ([B, W]), computed (i32). Outputs: out (bf16 bits), corr,
// decay (f32), key (bf16 bits), the committed state (f32), the compacted conv
// states (bf16 bits) and the plan arrays (i32).
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <map>
#include <string>
#include <vector>

#include "gdn_recoverssm_hip.h"

#define HIP_OK(x)                                                                      \
  do {                                                                                 \
    hipError_t e_ = (x);                                                               \
    if (e_ != hipSuccess) {                                                            \
      std::fprintf(stderr, "%s failed: %s\n", #x, hipGetErrorString(e_));              \
      std::exit(3);                                                                    \
    }                                                                                  \
  } while (0)

static void abi_ok(int status, const char *what) {
  if (status != GDN_OK) {
    std::fprintf(stderr, "%s returned %d: %s\n", what, status, gdn_recoverssm_last_error());
    std::exit(4);
  }
}

static std::vector<char> read_file(const std::string &path, size_t bytes) {
  std::vector<char> buf(bytes);
  FILE *f = std::fopen(path.c_str(), "rb");
  if (!f || std::fread(buf.data(), 1, bytes, f) != bytes) {
    std::fprintf(stderr, "cannot read %zu bytes from %s\n", bytes, path.c_str());
    std::exit(2);
  }
  std::fclose(f);
  return buf;
}

static void write_file(const std::string &path, const void *data, size_t bytes) {
  FILE *f = std::fopen(path.c_str(), "wb");
  if (!f || std::fwrite(data, 1, bytes, f) != bytes) {
    std::fprintf(stderr, "cannot write %s\n", path.c_str());
    std::exit(2);
  }
  std::fclose(f);
}

// A device copy of <dir>/<name>.bin (bytes long).
static void *upload(const std::string &dir, const char *name, size_t bytes) {
  std::vector<char> host = read_file(dir + "/" + name + ".bin", bytes);
  void *dev = nullptr;
  HIP_OK(hipMalloc(&dev, bytes));
  HIP_OK(hipMemcpy(dev, host.data(), bytes, hipMemcpyHostToDevice));
  return dev;
}

static void *zeros(size_t bytes) {
  void *dev = nullptr;
  HIP_OK(hipMalloc(&dev, bytes));
  HIP_OK(hipMemset(dev, 0, bytes));
  return dev;
}

static void download(const std::string &dir, const char *name, const void *dev, size_t bytes) {
  std::vector<char> host(bytes);
  HIP_OK(hipMemcpy(host.data(), dev, bytes, hipMemcpyDeviceToHost));
  write_file(dir + "/" + name + ".bin", host.data(), bytes);
}

int main(int argc, char **argv) {
  if (argc != 2) {
    std::fprintf(stderr, "usage: %s <dir>\n", argv[0]);
    return 2;
  }
  const std::string dir = argv[1];
  std::map<std::string, double> m;
  {
    FILE *f = std::fopen((dir + "/meta.txt").c_str(), "r");
    if (!f) {
      std::fprintf(stderr, "no meta.txt in %s\n", dir.c_str());
      return 2;
    }
    char key[64];
    double val;
    while (std::fscanf(f, "%63s %lf", key, &val) == 2) m[key] = val;
    std::fclose(f);
  }
  const int64_t B = int64_t(m["B"]), T = int64_t(m["T"]), H = int64_t(m["H"]), HV = int64_t(m["HV"]);
  const int64_t K = int64_t(m["K"]), V = int64_t(m["V"]), Q = int64_t(m["Q"]), NB = int64_t(m["NB"]);
  const int64_t W = int64_t(m["W"]), BS = int64_t(m["BS"]), CD = int64_t(m["CD"]), CW = int64_t(m["CW"]);
  const float scale = float(m["SCALE"]);
  if (gdn_recoverssm_abi_version() != 1) {
    std::fprintf(stderr, "ABI version %d\n", gdn_recoverssm_abi_version());
    return 4;
  }

  void *q = upload(dir, "q", size_t(T * H * K * 2));
  void *k = upload(dir, "k", size_t(T * H * K * 2));
  void *v = upload(dir, "v", size_t(T * HV * V * 2));
  void *g = upload(dir, "g", size_t(T * HV * 4));
  void *beta = upload(dir, "beta", size_t(T * HV * 4));
  void *state = upload(dir, "state", size_t(NB * HV * V * K * 4));
  void *conv = upload(dir, "conv", size_t(NB * CD * CW * 2));
  void *qsl = upload(dir, "qsl", size_t((B + 1) * 4));
  void *idx = upload(dir, "idx", size_t(B * 4));
  void *accepted = upload(dir, "accepted", size_t(B * 4));
  void *table = upload(dir, "table", size_t(B * W * 4));
  void *computed = upload(dir, "computed", size_t(B * 4));
  void *out = zeros(size_t(T * HV * V * 2));
  void *corr = zeros(size_t(B * HV * Q * V * 4));
  void *key = zeros(size_t(B * H * Q * K * 2));
  void *decay = zeros(size_t(B * HV * Q * 4));
  hipStream_t stream;
  HIP_OK(hipStreamCreate(&stream));

  // Verify: the 28 fields of the reference's GDN_VERIFY_FIELDS, contiguous
  // tensors, typed-SoA records (correction [B,HV,Q,V], key [B,H,Q,K], decay [B,HV,Q]).
  const int64_t vcfg[GDN_VERIFY_CONFIG_FIELDS] = {
      B, T, H, HV, Q, NB, B, 0,            // rows, tokens, heads, value heads, Q, blocks, record rows, null block
      H * K, H * K, HV * V, HV, HV,        // q, k, v, g, beta token strides
      HV * V * K, V * K, K,                // state block / head / row strides
      HV * Q * V, Q * V, V,                // correction row / head / token strides
      H * Q * K, Q * K, K,                 // key
      HV * Q, Q, 1,                        // decay
      HV * V, 1, 1,                        // out token stride, qsl and index strides
  };
  gdn_verify_ext vext{};
  vext.key_dim = K;
  vext.value_dim = V;
  vext.act_dtype = GDN_DT_BF16;
  vext.beta_dtype = GDN_DT_F32;
  vext.g_dtype = GDN_DT_F32;
  vext.state_dtype = GDN_DT_F32;
  vext.key_record_dtype = GDN_DT_BF16;
  vext.qsl_dtype = GDN_DT_I32;
  vext.index_dtype = GDN_DT_I32;
  vext.qk_l2norm = 0;
  vext.key_per_value_head = 0;
  vext.out_dtype = GDN_DT_BF16;
  abi_ok(gdn_recoverssm_verify(q, k, v, g, beta, state, corr, key, decay, out, qsl, idx, vcfg,
                               GDN_VERIFY_CONFIG_FIELDS, scale, &vext, stream),
         "gdn_recoverssm_verify");

  // Commit: plan + fold in one launch (align mode, one group, no request
  // mapping), then the conv compaction reading the plan it stored.
  int32_t *plan[7];
  for (auto &p : plan) p = static_cast<int32_t *>(zeros(size_t(B * 4)));
  gdn_plan_group grp{};
  grp.state_indices = idx;
  grp.si_stride = 1;
  grp.si_dtype = GDN_DT_I32;
  grp.query_start_loc = qsl;
  grp.qsl_stride = 1;
  grp.qsl_dtype = GDN_DT_I32;
  grp.block_table = table;
  grp.table_row_stride = W;
  grp.table_col_stride = 1;
  grp.table_width = W;
  grp.table_rows = B;
  grp.table_dtype = GDN_DT_I32;
  grp.num_computed = computed;
  grp.computed_stride = 1;
  grp.computed_len = B;
  grp.computed_dtype = GDN_DT_I32;
  grp.num_blocks = NB;
  grp.block_size = BS;
  gdn_plan_launch pl{};
  pl.sampled = accepted;
  pl.sampled_stride = 1;
  pl.sampled_len = B;
  pl.sampled_dtype = GDN_DT_I32;
  pl.num_groups = 1;
  pl.groups = &grp;
  pl.source_plan = plan[0];
  pl.lens_plan = plan[1];
  pl.final_plan = plan[2];
  pl.boundary_plan = plan[3];
  pl.boundary_lens_plan = plan[4];
  pl.valid_plan = plan[5];
  pl.col_plan = plan[6];
  pl.num_rows = B;
  pl.plan_capacity = B;
  pl.null_block = 0;
  pl.spec_query_len = Q;
  pl.flags = GDN_PLAN_ALIGN;
  // Per-layer tables (one layer), on the device: base addresses and block
  // strides of state, corrections, keys and decays, then the conv states'
  // base address and block / dim / token strides.
  const int64_t host_tables[12] = {reinterpret_cast<int64_t>(state), HV * V * K, reinterpret_cast<int64_t>(corr),
                                   HV * Q * V, reinterpret_cast<int64_t>(key), H * Q * K,
                                   reinterpret_cast<int64_t>(decay), HV * Q, reinterpret_cast<int64_t>(conv),
                                   CD * CW, CW, 1};
  int64_t *tables = nullptr;
  HIP_OK(hipMalloc(&tables, sizeof(host_tables)));
  HIP_OK(hipMemcpy(tables, host_tables, sizeof(host_tables), hipMemcpyHostToDevice));
  // The 17 fields of the reference's GDN_FOLD_FIELDS.
  const int64_t fcfg[GDN_FOLD_CONFIG_FIELDS] = {B, 1, HV, H, Q, NB, B, B, 0, V * K, K, Q * V, V, Q * K, K, Q, 1};
  gdn_fold_ext fext{};
  fext.key_dim = K;
  fext.value_dim = V;
  fext.state_dtype = GDN_DT_F32;
  fext.key_dtype = GDN_DT_BF16;
  fext.source_dtype = GDN_DT_I32;
  fext.source_stride = 1;
  fext.state_k_stride = 1;
  abi_ok(gdn_recoverssm_plan_fold(&pl, state, corr, key, decay, tables + 0, tables + 1, tables + 2, tables + 3,
                                  tables + 4, tables + 5, tables + 6, tables + 7, nullptr, fcfg,
                                  GDN_FOLD_CONFIG_FIELDS, &fext, stream),
         "gdn_recoverssm_plan_fold");
  abi_ok(gdn_recoverssm_conv_compact(tables + 8, tables + 9, tables + 10, tables + 11, idx, GDN_DT_I32, 1, plan[1],
                                     plan[2], plan[3], plan[4], nullptr, B, 0, B, 1, CD, CW - Q + 1, CW, NB, 2, 1,
                                     stream),
         "gdn_recoverssm_conv_compact");
  HIP_OK(hipStreamSynchronize(stream));

  download(dir, "out_out", out, size_t(T * HV * V * 2));
  download(dir, "out_corr", corr, size_t(B * HV * Q * V * 4));
  download(dir, "out_key", key, size_t(B * H * Q * K * 2));
  download(dir, "out_decay", decay, size_t(B * HV * Q * 4));
  download(dir, "out_state", state, size_t(NB * HV * V * K * 4));
  download(dir, "out_conv", conv, size_t(NB * CD * CW * 2));
  const char *plan_names[7] = {"out_source", "out_lens", "out_final", "out_boundary", "out_blen", "out_valid",
                               "out_col"};
  for (int i = 0; i < 7; ++i) download(dir, plan_names[i], plan[i], size_t(B * 4));
  std::printf("capi_step: B=%lld T=%lld HV=%lld K=%lld V=%lld Q=%lld done\n", (long long)B, (long long)T,
              (long long)HV, (long long)K, (long long)V, (long long)Q);
  HIP_OK(hipStreamDestroy(stream));
  return 0;
}
