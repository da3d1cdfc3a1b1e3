/*
 * gdn_recoverssm_hip.h -- C ABI of the MI355X (gfx950) RecoverSSM kernels.
 *
 * Plain pointers, sizes and a hipStream_t (passed as void*); no torch types.
 * Every entry point validates its arguments on the host and returns a status
 * code BEFORE anything is launched when they are invalid (the message is kept
 * in gdn_recoverssm_last_error()). Launches are asynchronous on `stream`, with
 * no host synchronisation, no allocation and no extra stream, so they can be
 * captured into a HIP graph.
 *
 * Reference interfaces each entry point replaces (paths inside the reference
 * plugin, plugin/gdn_recoverssm_ascend):
 *   gdn_recoverssm_abi_version   -> csrc/ops.cpp:244   abi_version() -> 1
 *   gdn_recoverssm_verify        -> csrc/ops.cpp:87-154, schema :245
 *                                   (and the Triton launch kernels.py:867-928)
 *   gdn_recoverssm_fold          -> csrc/ops.cpp:170-239, schema :246
 *                                   (and grouped_commit.py:837-892, kernels.py:1976-2047)
 *   gdn_recoverssm_plan          -> grouped_commit.py:741-799 (_grouped_plan_kernel)
 *                                   and kernels.py:1892-1928 (_prepare_commit_plan_kernel)
 *   gdn_recoverssm_conv_compact  -> grouped_commit.py:800-836, kernels.py:1931-1973
 *   gdn_recoverssm_publish       -> grouped_commit.py:531-610 (_publish_grouped_align_kernel)
 *   gdn_recoverssm_verify_gated  -> the gated verify of docs/reference/recoverssm_gdn_upstream.py:83-151
 *                                   (gating and q/k L2 norm fused into verify; the producers it
 *                                   replaces are called at spec_forward.py:91-96)
 *   gdn_recoverssm_verify_deferred -> the "deferred commit" of docs/GDN-RecoverSSM-实现方案.md:515-527,
 *                                   563-568: the fold (csrc/ops.cpp:170-239) applied inside the
 *                                   next step's verify
 *   gdn_recoverssm_set_state_cache_retain -> no counterpart: a cache hint for the verify launches
 *   gdn_recoverssm_settle        -> no counterpart: which pending rows of a deferred commit a
 *                                   settle folds (the next verifies do not apply them)
 */
#ifndef GDN_RECOVERSSM_HIP_H
#define GDN_RECOVERSSM_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GDN_RECOVERSSM_ABI_VERSION 1

/* Status codes. */
#define GDN_OK 0
#define GDN_ERR_INVALID 1     /* geometry / dtype / stride violation; nothing launched */
#define GDN_ERR_UNSUPPORTED 2 /* outside what this library implements; nothing launched */
#define GDN_ERR_LAUNCH 3      /* the HIP runtime rejected the launch */

/* Element type codes for tensors whose dtype is not fixed by the ABI. */
#define GDN_DT_F32 0
#define GDN_DT_BF16 1
#define GDN_DT_F16 2
#define GDN_DT_I32 3
#define GDN_DT_I64 4

/* Verify tiling: exactly the 28 integer fields of the reference's
 * GDN_VERIFY_FIELDS in csrc/common.h:8-36, in that order (strides in elements),
 * followed by the float scale (csrc/common.h:52-55). */
#define GDN_VERIFY_CONFIG_FIELDS 28
/* Fold tiling: the 17 fields of GDN_FOLD_FIELDS, csrc/common.h:37-54. */
#define GDN_FOLD_CONFIG_FIELDS 17

/* What this library adds over the reference's K=V=128 native specialisation
 * (csrc/ops.cpp:100-141): dimensions, dtypes and layout flags that the
 * reference's Triton kernel took as constexprs (kernels.py:534-545). */
typedef struct gdn_verify_ext {
  int64_t key_dim;          /* K (<= 256; a multiple of 4 for FP32 state, of 8 for 16-bit state) */
  int64_t value_dim;        /* V (>= 1) */
  int32_t act_dtype;        /* q, k, v, out: F32 / BF16 / F16 */
  int32_t beta_dtype;       /* activation dtype or F32 */
  int32_t g_dtype;          /* activation dtype or F32 */
  int32_t state_dtype;      /* checkpoint: F32 / BF16 / F16 */
  int32_t key_record_dtype; /* key record: F32 / BF16 / F16 */
  int32_t qsl_dtype;        /* query_start_loc: I32 / I64 */
  int32_t index_dtype;      /* state_indices: I32 / I64 */
  int32_t qk_l2norm;        /* 1: normalise q and k in-kernel (eps 1e-6), kernels.py:645-648 */
  int32_t key_per_value_head; /* 1: packed record layout, one key per value head, kernels.py:687-697 */
  int32_t out_dtype;        /* out: F32 / BF16 / F16 (kernels.py:657 stores in out's own dtype) */
  int64_t state_cache_retain; /* no counterpart in the reference: this call's cache hint, the bytes
                                 of state read with ordinary loads from the end of the batch (see
                                 gdn_recoverssm_set_state_cache_retain); 0: the process-wide
                                 setting; negative: none (every row non-temporal). Results do not
                                 depend on it. gdn_recoverssm_verify_deferred ignores it. */
} gdn_verify_ext;

typedef struct gdn_fold_ext {
  int64_t key_dim;       /* K */
  int64_t value_dim;     /* V */
  int32_t state_dtype;   /* F32 / BF16 / F16 */
  int32_t key_dtype;     /* F32 / BF16 / F16 */
  int32_t source_dtype;  /* I32 / I64: dtype of `source` */
  int32_t reserved;
  int64_t source_stride; /* element stride of `source` (1 for plan arrays; the
                            table-column stride when the single-context commit
                            reads state_indices directly, kernels.py:1229) */
  int64_t state_k_stride;/* must be 1 */
  /* No counterpart in the reference: gdn_recoverssm_fold only (NULL for every
   * other entry point). When row_list is not NULL, the launch folds only the
   * plan rows it lists: a device int32 array of row_list_len entries
   * (1 <= row_list_len <= rows), strictly increasing; an entry outside
   * [0, rows) or not greater than the entry before it folds nothing, so no row
   * is ever folded twice. The grid then covers layers x row_list_len x heads
   * instead of every row, which is what a flush of a few rows (requests that
   * left a deferred batch) costs. When row_count is not NULL as well (a device
   * int32 the device wrote, e.g. by gdn_recoverssm_settle), only the first
   * min(*row_count, row_list_len) entries are folded, by a fixed grid of at
   * most GDN_FOLD_LISTED_GRID workgroups that take the (layer, listed row,
   * head) tiles in turn: a list the host cannot size costs the tiles it
   * names, not a launch over every row. */
  const int32_t *row_list;
  int64_t row_list_len;
  const int32_t *row_count;
} gdn_fold_ext;

#define GDN_FOLD_LISTED_GRID 512

int gdn_recoverssm_abi_version(void);

/* Message of the calling thread's last failed call ("" before any failure); a
 * successful call leaves it unchanged, so read it only after a non-zero status. */
const char *gdn_recoverssm_last_error(void);

/* Speculative verify from the read-only checkpoint (kernels.py:491-697).
 * q, k: [1, T, H, K]; v, out: [1, T, HV, V]; g, beta: [T, HV] (head stride 1);
 * state: [blocks, HV, V, K] (K stride 1, never written); correction [R, HV, Q, V]
 * f32; key [R, H, Q, K] (or [R, HV, Q, K]-strided views in packed layout);
 * decay [R, HV, Q] f32; qsl [rows + 1]; indices [rows] (any element stride). */
int gdn_recoverssm_verify(const void *q, const void *k, const void *v, const void *g, const void *beta,
                          const void *state, void *correction, void *key, void *decay, void *out,
                          const void *qsl, const void *indices, const int64_t *config, int64_t config_len,
                          float scale, const gdn_verify_ext *ext, void *stream);

/* Gating fused into verify (docs/reference/recoverssm_gdn_upstream.py:135-151):
 * per token and value head, from the raw projections a and b,
 *   g    = -exp(A_log[hv]) * softplus(a + dt_bias[hv]),
 *   beta = sigmoid(b),
 * with softplus(x) = log(1 + exp(sb*x)) / sb when sb*x <= threshold, else x
 * (vLLM's fused_gdn_gating: sb = 1, threshold = 20), evaluated in FP32. */
typedef struct gdn_gating_ext {
  int32_t a_log_dtype;        /* A_log [HV]: F32 / BF16 / F16 */
  int32_t dt_bias_dtype;      /* dt_bias [HV]: F32 / BF16 / F16 */
  float softplus_beta;        /* > 0 */
  float softplus_threshold;
} gdn_gating_ext;

/* Verify with the gating producer fused in: identical to gdn_recoverssm_verify
 * except that `a` and `b` (token stride in config fields 11 and 12, dtypes in
 * ext->g_dtype and ext->beta_dtype) are the raw gate projections and A_log /
 * dt_bias are per-value-head parameters. Pair it with ext->qk_l2norm = 1 to
 * fuse the q/k normalisation as well. The decay record holds exp(g). */
int gdn_recoverssm_verify_gated(const void *q, const void *k, const void *v, const void *a, const void *b,
                                const void *a_log, const void *dt_bias, const void *state, void *correction,
                                void *key, void *decay, void *out, const void *qsl, const void *indices,
                                const int64_t *config, int64_t config_len, float scale, const gdn_verify_ext *ext,
                                const gdn_gating_ext *gating, void *stream);

/* The previous step's commit of one layer, left for the next verify to apply.
 * DEVICE arrays, int32: `rows` [current rows] gives for each row of the
 * current batch the PENDING row it continues (the row of the previous step's
 * plan and records; -1 or any value outside [0, num_rows) for none). The plan
 * arrays of that commit (source, accepted length, final, boundary, boundary
 * length; see gdn_recoverssm_plan) are indexed by pending row and cover
 * `num_rows` (>= 1) rows. The records are the previous step's typed SoA planes
 * (or packed FP32 rows, key_per_value_head = 1); they must not be the buffers
 * the current verify writes. No two current rows may continue the same
 * pending row (two requests never share a state page): both would fold it
 * into its final page. Strides in elements. */
typedef struct gdn_pending_commit {
  const int32_t *rows;
  const int32_t *source;
  const int32_t *lengths;
  const int32_t *final_indices;
  const int32_t *boundary_indices;
  const int32_t *boundary_lengths;
  const void *correction;     /* [R', HV, Q, V] FP32 */
  const void *key;            /* [R', H, Q, K] FP32 or the activation dtype */
  const void *decay;          /* [R', HV, Q] FP32 */
  int64_t record_rows;        /* R' */
  int64_t corr_strides[3];    /* row, head, token */
  int64_t key_strides[3];
  int64_t decay_strides[3];
  int32_t key_dtype;
  int32_t key_per_value_head;
  int64_t num_rows;           /* rows of the pending plan (the previous step's batch) */
} gdn_pending_commit;

/* Verify with the previous step's commit folded in (no counterpart entry in
 * the reference, whose design notes propose it). A current row applies the
 * pending commit of the row `rows` names when that commit is valid (accepted
 * length 1..Q, source and final pages in range) and the row's own state index
 * equals the commit's final page: the wave then reads the pending source page,
 * replays the accepted prefix exactly as gdn_recoverssm_fold does (FP32
 * arithmetic, stores rounded to the state type), stores the result to the
 * final page (and the boundary snapshot), and verifies the current window
 * from the folded state as stored. Every other row verifies from its own
 * state index as gdn_recoverssm_verify does, and a pending commit no current
 * row applies stays pending: flush it with gdn_recoverssm_fold before its
 * pages are reused. Rows must not share pages. With no token in the batch the
 * launch still applies the pending commits (q, k, v, g, beta and out may then
 * be NULL). */
int gdn_recoverssm_verify_deferred(const void *q, const void *k, const void *v, const void *g, const void *beta,
                                   const void *state, void *correction, void *key, void *decay, void *out,
                                   const void *qsl, const void *indices, const int64_t *config,
                                   int64_t config_len, float scale, const gdn_verify_ext *ext,
                                   const gdn_pending_commit *pending, void *stream);

/* Default of gdn_recoverssm_set_state_cache_retain: 64 MiB, measured best for
 * the verifies of a model's decode step, where no commit re-reads a layer's
 * pages right after its verify (the commit comes after every layer). */
#define GDN_STATE_CACHE_RETAIN_DEFAULT (64LL << 20)

/* No counterpart in the reference (a cache hint of this implementation).
 * How many bytes of checkpoint state a verify launch (gdn_recoverssm_verify,
 * gdn_recoverssm_verify_gated) reads with ordinary loads, counted from the end
 * of its batch: the rows before them read their pages non-temporally. What
 * the ordinary loads leave in the memory-side (Infinity) cache, 256 MB on
 * MI355X, is what a commit reading the same pages right after the verify
 * finds there (a single layer's verify, sampling, commit: retaining 256 MiB
 * suits it); in a decode step nothing re-reads them soon, and a quarter of a
 * B=128 layer's pages read ordinarily measured fastest. gdn_recoverssm_verify_deferred
 * reads and writes every row non-temporally whatever the setting. Results do
 * not depend on it. Process-wide, used by calls whose gdn_verify_ext leaves
 * state_cache_retain at 0; returns the previous value, or -1 (nothing
 * changed) for a negative `bytes`. */
int64_t gdn_recoverssm_set_state_cache_retain(int64_t bytes);

/* Grouped fold of the accepted prefix into every layer's checkpoint
 * (grouped_commit.py:377-480; csrc/fold.h:192-237). All table arguments are
 * DEVICE pointers: per-layer int64 base addresses / block strides [layers],
 * int32 layer_groups [layers] (may be NULL: every layer uses group 0), and the
 * int32 plan arrays [groups * plan_capacity]. state_ref/correction_ref/key_ref/
 * decay_ref are the first layer's tensors (unused for addressing, as in the
 * reference, csrc/fold.h:253-273). A row's source, final and boundary pages
 * may coincide; pages of different rows must not (one row's stores are not
 * ordered against another row's loads, as with the reference's kernels). */
int gdn_recoverssm_fold(void *state_ref, const void *correction_ref, const void *key_ref, const void *decay_ref,
                        const int64_t *state_addrs, const int64_t *state_block_strides, const int64_t *corr_addrs,
                        const int64_t *corr_block_strides, const int64_t *key_addrs,
                        const int64_t *key_block_strides, const int64_t *decay_addrs,
                        const int64_t *decay_block_strides, const int32_t *layer_groups, const void *source,
                        const int32_t *lengths, const int32_t *final_indices, const int32_t *boundary_indices,
                        const int32_t *boundary_lengths, const int64_t *config, int64_t config_len,
                        const gdn_fold_ext *ext, void *stream);

/* One cache group of the commit plan (grouped_commit.py:113-146). Pointers are
 * device pointers; request_indices may be NULL (row i is request i, the
 * single-context plan of kernels.py:979-983); block_table / num_computed are
 * NULL in "none" mode. *_len fields bound every index the kernel derives from
 * data: an index outside them makes the row invalid instead of reading out of
 * bounds. */
#define GDN_PLAN_MAX_GROUPS 8
typedef struct gdn_plan_group {
  const void *state_indices;   int64_t si_stride;       int32_t si_dtype;       int32_t pad0;
  const void *query_start_loc; int64_t qsl_stride;      int32_t qsl_dtype;      int32_t pad1;
  const void *request_indices; int64_t map_stride;      int32_t map_dtype;      int32_t pad2;
  const void *block_table;     int64_t table_row_stride; int64_t table_col_stride; int64_t table_width;
  int64_t table_rows;          int32_t table_dtype;     int32_t pad3;
  const void *num_computed;    int64_t computed_stride; int64_t computed_len;  int32_t computed_dtype; int32_t pad4;
  int64_t num_blocks;          int64_t block_size;
} gdn_plan_group;

#define GDN_PLAN_ALIGN 1u     /* align mode: block_table / num_computed present */
#define GDN_PLAN_PUBLISH 2u   /* publish persistent_cols / persistent_accepted (grouped_commit.py:214-222) */
#define GDN_PLAN_GROUPED 4u   /* grouped semantics: store the source, canonicalise the boundary
                                 (grouped_commit.py:194-204); without it the single-context
                                 semantics of kernels.py:1036-1072 apply */

int gdn_recoverssm_plan(const void *sampled, int32_t sampled_dtype, int64_t sampled_stride, int64_t sampled_len,
                        const gdn_plan_group *groups, int32_t num_groups, int32_t *source_plan,
                        int32_t *lens_plan, int32_t *final_plan, int32_t *boundary_plan,
                        int32_t *boundary_lens_plan, int32_t *valid_plan, int32_t *col_plan,
                        const void *idx_mapping, int32_t idx_mapping_dtype, int64_t idx_mapping_len,
                        int32_t *persistent_cols, int32_t *persistent_accepted, int64_t persistent_len,
                        int64_t num_rows, int64_t plan_capacity, int64_t null_block, int64_t spec_query_len,
                        uint32_t flags, void *stream);

/* The arguments of gdn_recoverssm_plan as one block, for the fused plan + fold
 * entry below (same meaning, same checks). */
typedef struct gdn_plan_launch {
  const void *sampled;
  int64_t sampled_stride;
  int64_t sampled_len;
  int32_t sampled_dtype;
  int32_t num_groups;
  const gdn_plan_group *groups; /* HOST pointer to num_groups entries */
  int32_t *source_plan, *lens_plan, *final_plan, *boundary_plan, *boundary_lens_plan, *valid_plan, *col_plan;
  const void *idx_mapping;
  int64_t idx_mapping_len;
  int32_t idx_mapping_dtype;
  uint32_t flags;
  int32_t *persistent_cols, *persistent_accepted;
  int64_t persistent_len;
  int64_t num_rows, plan_capacity, null_block, spec_query_len;
} gdn_plan_launch;

/* Plan and fold in one launch (no counterpart entry in the reference, which
 * launches its plan and fold kernels one after the other: kernels.py:1036-1072
 * then :1222-1324, grouped_commit.py:377-480). Every fold workgroup plans its
 * own (group, row) from the step's metadata and starts streaming the source
 * page before the block-table lookups return; extra workgroups store the plan
 * arrays (and the align publication) exactly as gdn_recoverssm_plan does, for
 * the conv compaction that follows. Results are identical to
 * gdn_recoverssm_plan followed by gdn_recoverssm_fold reading the plan it
 * stored (`source` = the group's state indices, or the plan's source for a
 * grouped plan). The fold arguments are those of gdn_recoverssm_fold without
 * the plan arrays; config[0] (rows) must equal plan->num_rows and config[7]
 * (capacity) plan->plan_capacity. */
int gdn_recoverssm_plan_fold(const gdn_plan_launch *plan, void *state_ref, const void *correction_ref,
                             const void *key_ref, const void *decay_ref, const int64_t *state_addrs,
                             const int64_t *state_block_strides, const int64_t *corr_addrs,
                             const int64_t *corr_block_strides, const int64_t *key_addrs,
                             const int64_t *key_block_strides, const int64_t *decay_addrs,
                             const int64_t *decay_block_strides, const int32_t *layer_groups,
                             const int64_t *config, int64_t config_len, const gdn_fold_ext *ext, void *stream);

/* Conv-state tables of one commit, for gdn_recoverssm_commit_noalloc: the
 * per-layer DEVICE tables and sizes of gdn_recoverssm_conv_compact below. */
typedef struct gdn_conv_launch {
  const int64_t *conv_addrs;
  const int64_t *conv_block_strides;
  const int64_t *conv_dim_strides;
  const int64_t *conv_token_strides;
  int64_t conv_dim;
  int64_t history;
  int64_t window;
  int32_t element_bytes;
  int32_t reserved;
} gdn_conv_launch;

/* Plan-array entries (plan->num_groups * plan->plan_capacity) that
 * gdn_recoverssm_commit_noalloc holds: 8 groups of 4096 rows. */
#define GDN_NOALLOC_PLAN_ENTRIES 32768

/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, serving loops that forbid hipMalloc):
 * the commit of gdn_recoverssm_plan_fold followed by gdn_recoverssm_conv_compact
 * (when `conv` is not NULL), with the seven plan arrays held in a buffer the
 * library owns on each GPU (7 x GDN_NOALLOC_PLAN_ENTRIES int32, 896 KiB,
 * kept until the process ends) instead of arrays the caller allocates. The
 * plan-array pointers of `plan` must be NULL; everything else has the meaning
 * and the checks of gdn_recoverssm_plan_fold (and of the conv compaction, with
 * config[1] layers and config[5] blocks), and pages, conv states and the align
 * publication come out identical. num_groups * plan_capacity above
 * GDN_NOALLOC_PLAN_ENTRIES is rejected before anything runs. The plan stays in
 * the library, so publication across buckets (gdn_recoverssm_publish) is not
 * available through this entry; GDN_PLAN_PUBLISH within one plan is. Every
 * call on a GPU shares that GPU's buffer: calls that overlap on one GPU (on
 * different streams, or from different threads without ordering) race. The
 * stream must belong to the current device. Nothing is allocated: the first
 * call on a device only looks the buffer's address up. */
int gdn_recoverssm_commit_noalloc(const gdn_plan_launch *plan, void *state_ref, const void *correction_ref,
                                  const void *key_ref, const void *decay_ref, const int64_t *state_addrs,
                                  const int64_t *state_block_strides, const int64_t *corr_addrs,
                                  const int64_t *corr_block_strides, const int64_t *key_addrs,
                                  const int64_t *key_block_strides, const int64_t *decay_addrs,
                                  const int64_t *decay_block_strides, const int32_t *layer_groups,
                                  const int64_t *config, int64_t config_len, const gdn_fold_ext *ext,
                                  const gdn_conv_launch *conv, void *stream);

/* Conv-state compaction (grouped_commit.py:225-322 / kernels.py:1075-1169).
 * Per-layer DEVICE tables: base addresses, block / dim / token strides
 * (elements). element_bytes is 2 or 4. `source` as in gdn_recoverssm_fold.
 * history is the kept history length, window the conv state's token extent
 * (history + Q - 1); every token read stays inside the window. Only the first
 * `history` positions of the final (and boundary) slot change; slots of
 * different rows must not coincide, as for gdn_recoverssm_fold. */
int gdn_recoverssm_conv_compact(const int64_t *conv_addrs, const int64_t *conv_block_strides,
                                const int64_t *conv_dim_strides, const int64_t *conv_token_strides,
                                const void *source, int32_t source_dtype, int64_t source_stride,
                                const int32_t *lengths, const int32_t *final_indices,
                                const int32_t *boundary_indices, const int32_t *boundary_lengths,
                                const int32_t *layer_groups, int64_t plan_capacity, int64_t null_block,
                                int64_t num_rows, int64_t num_layers, int64_t conv_dim, int64_t history,
                                int64_t window, int64_t num_blocks, int32_t element_bytes, int32_t align,
                                void *stream);

/* AND-valid publication across buckets (grouped_commit.py:531-560).
 * descriptors: DEVICE int64 [num_buckets * 4] = (valid ptr, col ptr, capacity,
 * group count) per bucket. request_len is the number of entries of
 * request_indices (at least num_rows). */
int gdn_recoverssm_publish(const int64_t *descriptors, int64_t num_buckets, const void *request_indices,
                           int32_t request_dtype, int64_t request_stride, int64_t request_len,
                           const void *idx_mapping, int32_t idx_mapping_dtype, int64_t idx_mapping_len,
                           int32_t *persistent_cols, int32_t *persistent_accepted, int64_t persistent_len,
                           int64_t num_rows, void *stream);

/* No counterpart in the reference: what a settle of a deferred commit folds,
 * decided on the device for the 1..GDN_SETTLE_MAX_GROUPS plan groups of one
 * plan (a commit context, or a bucket of cache groups). Group g's pending row
 * r < num_rows is applied by the next step's deferred verify when some next
 * row b < next[g].rows has rows[b] == r and next[g].state_indices[b *
 * next[g].stride] == finals[g * capacity + r] (the verify's own test). Then
 * out_lengths[g * capacity + r] = 0 for every applied row and lengths[...]
 * for every other entry (entries from num_rows on included), and row_list
 * receives, ascending, every r < num_rows whose out length is above 0 in some
 * group, *row_count their number: a gdn_recoverssm_fold of out_lengths with
 * that row list and count (gdn_fold_ext.row_list / row_count) commits
 * exactly the pending rows the next verifies will not apply. The plan's
 * length of every entry handed on that way (r < num_rows, out length above
 * 0) is set to 0, so a later settle or flush of the same plan does not fold
 * it again, while the rows the verifies apply keep theirs. lengths, finals
 * and out_lengths hold num_groups * capacity entries, row_list at least
 * max(num_rows, 1), rows (the next batch's row map: next row -> pending row,
 * -1 for a new request) at least the largest next[g].rows; `next` is a HOST
 * array of num_groups entries (rows 0: nothing of that group is applied).
 * One workgroup; num_rows is at most GDN_SETTLE_MAX_ROWS. The outputs share
 * memory with no input and with each other. */
#define GDN_SETTLE_MAX_GROUPS 3
#define GDN_SETTLE_MAX_ROWS 65536
typedef struct gdn_settle_next {
  const void *state_indices; /* DEVICE: the next batch's state index of row b at b * stride */
  int64_t stride;            /* element stride */
  int64_t rows;              /* next rows of this group */
  int32_t dtype;             /* GDN_DT_I32 / GDN_DT_I64 */
  int32_t reserved;
} gdn_settle_next;

int gdn_recoverssm_settle(int32_t *lengths, const int32_t *finals, int64_t num_groups, int64_t capacity,
                          int64_t num_rows, const int32_t *rows, int64_t rows_len, const gdn_settle_next *next,
                          int32_t *out_lengths, int32_t *row_list, int32_t *row_count, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* GDN_RECOVERSSM_HIP_H */
