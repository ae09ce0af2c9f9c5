/*
 * thundersync_hip.h -- C ABI of libthundersync_hip.so, the MI355X (gfx950)
 * kernels behind thundersync_amd's operators.
 *
 * Conventions (all entry points):
 *   - every tensor argument is a raw device pointer (except in the forest
 *     metadata section: host code over host arrays); sizes and strides are
 *     int64 element counts; `stream` is a hipStream_t passed as void*;
 *   - the caller (PyTorch on the host side) allocates every input, output
 *     and workspace; the library never allocates, frees or retains device
 *     memory (the host-side metadata builders use temporary host memory);
 *   - inputs are never written, so a call may be repeated on the same
 *     inputs (activation-checkpoint recompute does exactly that);
 *   - the return value is a status (TS_OK or a TS_ERR_* code); the message
 *     of the last failure on the calling thread is ts_hip_last_error().
 *
 * Each declaration names the reference interface it replaces.  Paths are
 * relative to the reference repository root (seilk/thundersync,
 * src/thundersync/...).
 */
#ifndef THUNDERSYNC_HIP_H
#define THUNDERSYNC_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TS_OK 0
#define TS_ERR_INVALID 1   /* bad argument: shape, dtype, alignment, size */
#define TS_ERR_LAUNCH 2    /* the HIP runtime refused a launch */
#define TS_ERR_DEVICE 3    /* the current device is not a gfx950 */

/* dtype codes */
#define TS_F32 0
#define TS_F16 1
#define TS_BF16 2
#define TS_F64 3

/* Library version string, e.g. "thundersync_hip 0.1.0 gfx950". */
const char* ts_hip_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* ts_hip_last_error(void);

/* ------------------------------------------------------------------------
 * RMSNorm
 * ------------------------------------------------------------------------ */

/* Forward with the replaced Qwen3RMSNorm's operation order and casts:
 *   xf = float(x); rstd = rsqrt(mean(xf^2) + eps);
 *   y = w * T(xf * rstd)            (product rounded to T, as torch does)
 * x, y: [rows, width] of dtype; w: [width] of dtype; rstd: [rows] fp32.
 * y and rstd are byte-identical to the stock module's on the GPU: mean(xf^2)
 * is summed in the order torch's reduction kernel uses for a contiguous
 * [rows, width] fp32 tensor on the device's CU count, and rsqrt is correctly
 * rounded, as torch.rsqrt is.  TS_ERR_INVALID for a single row wider than
 * 130560 (torch sums such a row across work-groups).
 * Replaces FP32RMSNormVJP.forward (accel/rms_norm.py:9-17) and the compiled
 * primal `_primal` / `_CompiledForwardVJP` (grpo/rms_norm.py:12-31). */
int ts_rmsnorm_fwd(const void* x, const void* w, void* y, float* rstd,
                   int64_t rows, int64_t width, float eps, int dtype,
                   void* stream);

/* 1 when ts_rmsnorm_fwd and ts_rmsnorm_bwd both take a contiguous
 * [rows, width] problem on the device `stream` belongs to, else 0 (a single
 * row that torch sums across work-groups; a width the backward has no kernel
 * for).  No launch, no allocation.  The module swap's eligibility test: the
 * reference's StableQwen3RMSNorm keeps the stock forward outside its own
 * path (accel/rms_norm.py:49-52), and the swap here does the same for the
 * shapes this returns 0 for. */
int ts_rmsnorm_supported(int64_t rows, int64_t width, void* stream);

/* Workspace bytes ts_rmsnorm_bwd needs for `rows` x `width`. */
int64_t ts_rmsnorm_bwd_workspace(int64_t rows, int64_t width);

/* FP32 VJP from the saved statistic:
 *   xhat = float(x) * rstd;  g = float(dy) * float(w)
 *   dx = T(rstd * (g - xhat * mean(g * xhat)))
 *   dw = T(sum_rows float(dy) * float(x) * rstd)
 * dx or dw may be NULL when that gradient is not needed.  The dw sum is a
 * fixed-order reduction: identical inputs give identical bits.
 * Replaces FP32RMSNormVJP.backward (accel/rms_norm.py:19-43, the
 * aten._fused_rms_norm_backward call at :28) and
 * native_source_rms_backward with its Triton dW kernels
 * (grpo/rms_norm_native.py:8-74). */
int ts_rmsnorm_bwd(const void* dy, const void* x, const void* w,
                   const float* rstd, void* dx, void* dw, void* workspace,
                   int64_t workspace_bytes, int64_t rows, int64_t width,
                   int dtype, void* stream);

/* Size of the device array ts_rmsnorm_bwd_noalloc keeps its dW partials in
 * (one per GPU the library runs on, held until the process ends). */
#define TS_RMSNORM_BWD_SCRATCH_BYTES (8 << 20)

/* ts_rmsnorm_bwd without a workspace argument and without any allocation:
 * the dW partials go to a file-scope device array of
 * TS_RMSNORM_BWD_SCRATCH_BYTES.  No counterpart in the reference; it is for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc).  TS_ERR_INVALID when
 * ts_rmsnorm_bwd_workspace(rows, width) exceeds the array (every row count
 * fits for width <= 8192).  All calls on one GPU share its array, so only one
 * caller per GPU may have a call in flight at a time: calls that overlap on
 * one GPU (two streams, two threads) race on the partials.  Results are
 * bit-identical to ts_rmsnorm_bwd's. */
int ts_rmsnorm_bwd_noalloc(const void* dy, const void* x, const void* w,
                           const float* rstd, void* dx, void* dw, int64_t rows,
                           int64_t width, int dtype, void* stream);

/* ------------------------------------------------------------------------
 * Forest / packed bottom-right-causal GQA attention (bf16 or fp16; head_dim
 * D = 32, 64, 96, 128, 192 or 256)
 *
 * A problem is a set of query SEGMENTS and key RUNS.  Segment s owns query
 * rows [q_row0, q_row0 + q_len) of the packed Q/O/dO/dQ tensors
 * ([rows, Hq, D], any row/head stride) and attends to a virtual key
 * sequence of kv_len keys assembled from runs: seg_spans[span0 .. span0 +
 * nspan) lists (run, kpos) -- run `index` supplies keys [kpos, kpos + len)
 * of that sequence.  Visibility is bottom-right causal over the sequence:
 * query row i sees key position j iff j <= kv_len - q_len + i.  A run is
 * one contiguous [len, Hkv, D] block of K/V rows (a retained chunk, a
 * forest node, a prefix), read in place through its own pointers and
 * strides, never concatenated; run_visits[visit0 .. visit0 + nvisit) lists
 * (segment, kpos) -- every segment that reads it -- and the backward writes
 * the run's dK/dV, summed over those visits, through its dk/dv pointers.
 *
 * This one description covers:
 *   - _causal_sdpa(query, ks, vs, scale) with ks/vs a chunk list: one
 *     segment, one run per chunk (engine/streaming.py:1080-1162);
 *   - _ChunkedCausalSDPA (retained per-chunk K/V, :1314-1423);
 *   - _PackedFlashSplit over a plain turn pack (:1704-1836): one segment per
 *     turn, its ancestor chunks and its own K/V as runs;
 *   - _ragged_causal_sdpa cohorts (:1165-1297);
 *   - forest_attention(q, k, v, plan) (engine/attention.py:186-231): one
 *     segment per node, one run per node, key_ranges as the span lists.
 * The split-at-the-prefix-plus-LSE-merge of the reference's flash/cuDNN
 * paths (:614-803, :939-1077) is not needed: each segment's softmax runs
 * over its whole key sequence in one pass.
 * ------------------------------------------------------------------------ */

typedef struct ts_attn_ref {
  int32_t index; /* run (in seg_spans) or segment (in run_visits) */
  int32_t kpos;  /* position of the run's first key in the segment's keys */
} ts_attn_ref;

typedef struct ts_attn_segment {
  int64_t q_row0;
  int32_t q_len;
  int32_t kv_len;
  int32_t span0;
  int32_t nspan;
} ts_attn_segment;

typedef struct ts_attn_run {
  uint64_t k, v;   /* device address of key 0, kv-head 0 */
  uint64_t dk, dv; /* gradient destinations (backward only; may be 0) */
  int64_t k_row_stride, k_head_stride, v_row_stride, v_head_stride;
  int64_t dk_row_stride, dk_head_stride, dv_row_stride, dv_head_stride;
  int32_t len;
  int32_t visit0;
  int32_t nvisit;
  int32_t reserved;
} ts_attn_run;

typedef struct ts_attn_problem {
  const ts_attn_segment* segs; /* device arrays */
  const ts_attn_ref* seg_spans;
  const ts_attn_run* runs;
  const ts_attn_ref* run_visits;
  const int32_t* q_work;  /* pairs (segment, first row): one per 32-row block */
  const int32_t* kv_work; /* pairs (run, first key): one per kv_block keys */
  int32_t n_q_work;
  int32_t n_kv_work;
  int32_t n_segs;
  int32_t n_runs;
  int32_t hq;
  int32_t hkv;
  int32_t head_dim; /* 32, 64, 96, 128, 192 or 256 */
  float scale;
  int32_t q_block;  /* rows per q_work item: ts_attn_q_block(hq / hkv) */
  int32_t kv_block; /* keys per kv_work item: ts_attn_kv_block(hq / hkv, head_dim) */
  int64_t q_rows;   /* rows of Q/O/dO/dQ */
  /* Launch order.  The work lists are sorted longest first; their first
   * n_q_long / n_kv_long items run first, item by item across all heads (so
   * no head's long item is left for the end of the launch), the rest head by
   * head (all XCDs then stream the same head's rows through the shared
   * last-level cache).  0 <= n_*_long <= n_*_work. */
  int32_t n_q_long;
  int32_t n_kv_long;
  int32_t dtype;  /* element type of Q/K/V/O/dO/dQ/dK/dV: TS_BF16 or TS_F16 */
} ts_attn_problem;

/* Query heads one forward/dQ work-group processes for a GQA group size
 * (hq / hkv): 4 when it divides the group, else 2, else 1. */
int ts_attn_heads_per_block(int group);

/* Query rows per forward/dQ work item for a GQA group size:
 * 32 * 4 / ts_attn_heads_per_block(group). */
int ts_attn_q_block(int group);

/* Keys per dK/dV work-group for a GQA group size and head dim: 48 when 4
 * divides the group below head dim 256 (one wave per query head), else 64.
 * At head dim 256 a problem may also hold 48-key items (the key-split
 * kernel, for launches with few work items). */
int ts_attn_kv_block(int group, int head_dim);

/* Host-side consistency check of a problem's tables, given as host copies
 * of the arrays the problem's device pointers name (those pointers are not
 * read): segment rows inside [0, q_rows) and kv_len >= q_len; each
 * segment's spans tile its keys in order over runs that exist; every run
 * non-empty, its K/V (and dK/dV, when set) 16-byte aligned with strides
 * that are multiples of 8 (row strides below 2^24), its visits in range and
 * each one a span of the segment it names, as many visits as spans; the work
 * lists hold every row block (q_block) of every segment and every key block
 * (kv_block) of every visited run exactly once; the long-item counts within
 * the lists.  TS_OK, or TS_ERR_INVALID naming the first inconsistency.  The
 * entry points trust the device tables; the Python layer runs this check
 * on every call's tables before they are uploaded.  No counterpart in the
 * reference (its tables are torch tensors checked by the flash kernels'
 * own argument checks). */
int ts_attn_check_tables(const ts_attn_problem* problem, const ts_attn_segment* segs,
                         const ts_attn_ref* seg_spans, int64_t n_spans, const ts_attn_run* runs,
                         const ts_attn_ref* run_visits, int64_t n_visits, const int32_t* q_work,
                         const int32_t* kv_work);

typedef struct ts_attn_rows {
  uint64_t ptr; /* device address of row 0, head 0 */
  int64_t row_stride;
  int64_t head_stride;
} ts_attn_rows;

/* Forward: out (bf16) and lse (fp32, natural log, [hq, lse_ld]).
 * Replaces the dispatch of _causal_sdpa (engine/streaming.py:1080-1162),
 * _flash_split_grouped_forward (:710-731), _PackedFlashSplit.forward
 * (:1727-1775), _ragged_causal_sdpa (:1165-1226), forest_attention
 * (engine/attention.py:186-231) and FA4's flash_attn_func(causal=True)
 * (:508-529). */
int ts_attn_fwd(const ts_attn_problem* problem, ts_attn_rows q, ts_attn_rows out,
                float* lse, int64_t lse_ld, void* stream);

/* Backward: dq (bf16, same row layout contract as q) and each run's dK/dV
 * (bf16, written through the run's dk/dv, summed over the run's visits in a
 * fixed order -- no atomics).  `rowstats` is a caller-provided fp32
 * workspace of 2 * hq * lse_ld floats: the backward writes, per (head, row),
 * the pair (lse * log2(e), rowsum(dO * O)) and reads it back.  q and dout
 * row strides must be below 2^25 elements and every run's K/V row stride
 * below 2^24 (byte offsets of a tile fit 32 bits).
 * Replaces _flash_split_grouped_backward (engine/streaming.py:734-768),
 * _ChunkedCausalSDPA.backward (:1378-1423), _PackedFlashSplit.backward and
 * its two varlen flash backward calls (:1777-1836), the per-segment
 * recompute of _RaggedAttentionIndependentVJP.backward (:1273-1297). */
int ts_attn_bwd(const ts_attn_problem* problem, ts_attn_rows q, ts_attn_rows out,
                ts_attn_rows dout, const float* lse, int64_t lse_ld, float* rowstats,
                ts_attn_rows dq, void* stream);

/* dS route of the backward.  ts_attn_bwd's dQ kernel recomputes S = Q K^T
 * and dP = dO V^T, which its dK/dV kernels also compute; on this route the
 * dK/dV kernels store dS = P (dP - delta) (in the element type, as rounded
 * for their own dK product) into a caller-provided workspace and the dQ
 * kernel forms dQ = scale dS K from it: the MFMA work of the backward drops
 * from 14 to 10 D flops per (row, key, head) for one write and one read of
 * 2 bytes per pair and head.  Same results contract as ts_attn_bwd
 * (deterministic, no atomics).
 *
 * ts_attn_ds_route(head_dim, group): 1 where the route exists (head dims
 * 128 and 256, every GQA group size hq / hkv); elsewhere ts_attn_bwd_ds runs
 * ts_attn_bwd's kernels and leaves the workspace untouched.
 *
 * ts_attn_ds_layout: the workspace layout of a set of tables (host copies;
 * run_len, visit0 and nvisit are the runs' len / visit0 / nvisit fields):
 * per span and per visit the element offset of that (segment, run) pair's
 * dS blocks within one head's part, and the elements of one head's part
 * (*ds_head).  Each pair takes 512 elements (32 rows x 16 keys) per block of
 * the keys its rows see, 2 bytes each: about 2 bytes per visible pair and
 * head.  TS_OK or TS_ERR_INVALID.
 *
 * ts_attn_bwd_ds: as ts_attn_bwd, with span_ds / visit_ds the device copies
 * of the layout's offsets and `ds` a 16-byte aligned device workspace of at
 * least (hq * ds_head + 512) * 2 bytes: every head's part, then one block
 * that takes the stores of steps that compute no dS (its contents on entry
 * do not matter).  dq_work (device; may be NULL): the dQ pass's own work
 * list for GQA groups that are a multiple of 4 at head dim 128, pairs
 * (segment, first row) of 64-row blocks (first row a multiple of 64, below
 * the segment's rows; every such block of every segment once, longest first
 * as the other lists, its first n_dq_long items item-major): each dQ
 * work-group then serves two 32-row blocks, sharing its K tiles between
 * eight waves instead of four.  NULL: the dQ pass takes the problem's
 * q_work.
 * No counterpart in the reference, whose flash/FA4 backward kernels own
 * their scratch; it replaces the same calls as ts_attn_bwd. */
int ts_attn_ds_route(int head_dim, int group);
int ts_attn_ds_layout(const ts_attn_segment* segs, int32_t n_segs, const ts_attn_ref* seg_spans,
                      int64_t n_spans, const int32_t* run_len, int32_t n_runs,
                      const ts_attn_ref* run_visits, const int32_t* visit0, const int32_t* nvisit,
                      int64_t n_visits, int64_t* span_ds, int64_t* visit_ds, int64_t* ds_head);
int ts_attn_bwd_ds(const ts_attn_problem* problem, ts_attn_rows q, ts_attn_rows out,
                   ts_attn_rows dout, const float* lse, int64_t lse_ld, float* rowstats,
                   ts_attn_rows dq, const int64_t* span_ds, const int64_t* visit_ds,
                   int64_t ds_head, void* ds, int64_t ds_bytes, const int32_t* dq_work,
                   int32_t n_dq_work, int32_t n_dq_long, void* stream);

/* ------------------------------------------------------------------------
 * Fused chunked-vocab logprob / entropy (bf16 or fp16 operands, fp32 results)
 *
 * hidden [rows, dim] (row stride ld_hidden), weight [vocab, dim] (ld_weight),
 * target int64 [rows]; hidden, weight, dlogits and grad_hidden share the
 * element type `dtype` (TS_BF16 or TS_F16).  dim and both leading dimensions are multiples of 8
 * and the bases 16-byte aligned; leading dimensions are below 2^30 / 255
 * elements (a 256-row tile's byte offsets fit 32 bits).  A target outside
 * [0, vocab) is not an error: its logprob is NaN and its dlogits row takes
 * no one-hot term.
 * ------------------------------------------------------------------------ */

/* Workspace bytes ts_logprob_fwd needs. */
int64_t ts_logprob_fwd_workspace(int64_t rows, int64_t vocab);

/* logprob[n] = l[n, target[n]] - lse[n] and, when `entropy` is not NULL,
 * entropy[n] = lse[n] - sum_v softmax(l[n])_v l[n, v], with l = hidden . W^T
 * accumulated in fp32 on MFMA; lse (natural log) is written for the backward.
 * A target outside [0, vocab) yields NaN.
 * Replaces _FusedLinearLogprob.forward and _FusedLinearLogprobEntropy.forward
 * (accel/fused_logprob.py:69-113, :249-267): its per-chunk fp32 [chunk, V]
 * logits, amax, logsumexp, gather and softmax passes. */
int ts_logprob_fwd(const void* hidden, int64_t ld_hidden, const void* weight,
                   int64_t ld_weight, const int64_t* target, int64_t rows,
                   int64_t dim, int64_t vocab, float* logprob, float* entropy,
                   float* lse, void* workspace, int64_t workspace_bytes,
                   int dtype, void* stream);

/* dlogits [rows, ld_dlogits] (bf16) =
 *   -p * (g_lp + g_ent * (log p + H)) + g_lp * onehot(target),
 * p = exp(l - lse), recomputing l on MFMA; columns [vocab, roundup8(vocab))
 * are written as zero.  grad_ent may be NULL (logprob-only objective).
 * Replaces the coefficient backward of _FusedLinearLogprob.backward and
 * _FusedLinearLogprobEntropy.backward (accel/fused_logprob.py:143-165,
 * :285-295): rematerialised logits, softmax, scatter_add and bf16 cast. */
int ts_logprob_dlogits(const void* hidden, int64_t ld_hidden, const void* weight,
                       int64_t ld_weight, const int64_t* target, const float* lse,
                       const float* entropy, const float* grad_lp,
                       const float* grad_ent, int64_t rows, int64_t dim,
                       int64_t vocab, void* dlogits, int64_t ld_dlogits,
                       int dtype, void* stream);

/* Workspace bytes ts_logprob_grad_hidden needs for rows x dim x vocab (0
 * when the row tiles alone fill the device and no vocabulary split is made). */
int64_t ts_logprob_grad_hidden_workspace(int64_t rows, int64_t dim, int64_t vocab);

/* grad_hidden [rows, dim] (bf16) = dlogits [rows, vocab] . W [vocab, dim],
 * fp32 accumulation on MFMA, W read in place (as the K-strided operand;
 * no transposed copy).  When the row tiles alone do not fill the device the
 * vocabulary is cut into ranges whose fp32 partial sums (the workspace) are
 * added in range order: deterministic.  Replaces the hidden VJP
 * `_matmul_accum(dlogits, weight)` of _FusedLinearLogprob.backward and
 * _FusedLinearLogprobEntropy.backward (accel/fused_logprob.py:167-175,
 * :297-303). */
int ts_logprob_grad_hidden(const void* dlogits, int64_t ld_dlogits, const void* weight,
                           int64_t ld_weight, int64_t rows, int64_t dim, int64_t vocab,
                           void* grad_hidden, int64_t ld_grad, void* workspace,
                           int64_t workspace_bytes, int dtype, void* stream);

/* grad_weight [vocab, ld_grad] (fp32) += dlogits[:rows]^T . hidden[:rows]
 * on MFMA with fp32 accumulation; called once per dlogits block, it
 * accumulates the weight gradient across blocks in block order, to be cast to
 * the weight dtype once (bf16 operands, as the reference's bf16 dlogits and
 * hidden).  Replaces `_matmul_accum(dlogits.t(), h)` and the fp32
 * `grad_weight.add_` of _FusedLinearLogprob.backward
 * (accel/fused_logprob.py:176-193, :304-306). */
int ts_logprob_grad_weight(const void* dlogits, int64_t ld_dlogits, const void* hidden,
                           int64_t ld_hidden, int64_t rows, int64_t dim, int64_t vocab,
                           float* grad_weight, int64_t ld_grad, int dtype, void* stream);

/* ------------------------------------------------------------------------
 * Fused logprob / entropy at the inputs' precision (fp32 or fp64)
 *
 * The reference keeps FP32/FP64 hidden states and heads at their precision
 * (accel/fused_logprob.py:27-58: `_accum_dtype` widens only bf16/fp16); these
 * entry points compute logits, softmax statistics, dlogits and both VJP
 * products in the input type T (dtype TS_F32 or TS_F64) on the vector ALUs.
 * hidden [rows, dim] (row stride ld_hidden), weight [vocab, dim]
 * (ld_weight), target int64 [rows]; every other array is of T.  No
 * alignment or stride-multiple requirements.  A target outside [0, vocab)
 * yields a NaN logprob and no one-hot term, as in the bf16/fp16 operators.
 * ------------------------------------------------------------------------ */

/* Workspace bytes ts_logprob_fwd_exact needs (-1 for a bad argument). */
int64_t ts_logprob_fwd_exact_workspace(int64_t rows, int64_t vocab, int dtype);

/* logprob[n] = l[n, target[n]] - lse[n], lse[n] (natural log) and, when
 * `entropy` is not NULL, entropy[n] = lse[n] - sum_v softmax(l[n])_v l[n, v],
 * with l = hidden . W^T, all in T.  Replaces _FusedLinearLogprob.forward and
 * _FusedLinearLogprobEntropy.forward for fp32/fp64 inputs
 * (accel/fused_logprob.py:69-113, :249-267). */
int ts_logprob_fwd_exact(const void* hidden, int64_t ld_hidden, const void* weight, int64_t ld_weight,
                         const int64_t* target, int64_t rows, int64_t dim, int64_t vocab, void* logprob,
                         void* entropy, void* lse, void* workspace, int64_t workspace_bytes, int dtype,
                         void* stream);

/* dlogits [rows, ld_dlogits] (T) = -p * (g_lp + g_ent * (log p + H)) +
 * g_lp * onehot(target), p = exp(l - lse), recomputing l; grad_ent (and
 * then entropy) may be NULL for the logprob-only objective.  Replaces the
 * coefficient backward of _FusedLinearLogprob.backward and
 * _FusedLinearLogprobEntropy.backward for fp32/fp64 inputs
 * (accel/fused_logprob.py:143-165, :285-295). */
int ts_logprob_dlogits_exact(const void* hidden, int64_t ld_hidden, const void* weight, int64_t ld_weight,
                             const int64_t* target, const void* lse, const void* entropy, const void* grad_lp,
                             const void* grad_ent, int64_t rows, int64_t dim, int64_t vocab, void* dlogits,
                             int64_t ld_dlogits, int dtype, void* stream);

/* c [m, n] (row stride ldc) = a . b, or c += a . b when accumulate != 0,
 * in T: element (i, j) of the product is sum_k a[i a_m + k a_k] *
 * b[k b_k + j b_n] (any element strides).  The hidden and weight VJPs
 * `_matmul_accum(dlogits, weight)` and `_matmul_accum(dlogits.t(), h)` with
 * the `grad_weight.add_` of _FusedLinearLogprob.backward for fp32/fp64
 * inputs (accel/fused_logprob.py:167-193, :297-306). */
int ts_matmul_exact(const void* a, int64_t a_m, int64_t a_k, const void* b, int64_t b_k, int64_t b_n, int64_t m,
                    int64_t n, int64_t k, void* c, int64_t ldc, int accumulate, int dtype, void* stream);

/* ------------------------------------------------------------------------
 * Merged-weight LoRA linear (bf16 or fp16 operands, fp32 accumulation)
 *
 * The caller has merged the adapters into the weight (W_eff = W + s B A,
 * [out, in]); lora_a is A [rank, in] and lora_b_t is B transposed,
 * [rank, out], both in the activations' dtype with rows of in / out
 * elements; `dtype` (TS_BF16 or TS_F16) is that of x, the weight, the
 * adapters, y, grad_out and grad_x.  Rows of x, y, g
 * and the weight are 16-byte aligned, in and out multiples of 8.
 * ------------------------------------------------------------------------ */

/* y [rows, out] = x [rows, in] . W_eff^T.
 * Replaces FusedLoRALinear.forward (accel/fused_lora.py:29-33). */
int ts_lora_fwd(const void* x, int64_t ld_x, const void* weight, int64_t ld_weight, int64_t rows,
                int64_t in_features, int64_t out_features, void* y, int64_t ld_y, int dtype, void* stream);

/* Workspace bytes ts_lora_bwd needs. */
int64_t ts_lora_bwd_workspace(int64_t rows, int64_t in_features, int64_t out_features, int64_t rank);

/* grad_x [rows, in] (bf16) = g W_eff; grad_a [rank, in] (fp32) =
 * s (g B)^T x; grad_b [out, rank] (fp32) = s g^T (x A^T), with g = grad_out
 * [rows, out].  g B and x A^T are rounded to bf16 (the reference forms them
 * as activation-dtype products); the adapter gradients are fp32 sums over
 * fixed row ranges added in range order, then scaled: the same bytes on
 * every call.  A null grad_x / grad_a / grad_b is not computed.  rank <= 256.
 * Replaces FusedLoRALinear.backward (accel/fused_lora.py:35-48). */
int ts_lora_bwd(const void* grad_out, int64_t ld_grad_out, const void* x, int64_t ld_x, const void* weight,
                int64_t ld_weight, const void* lora_a, const void* lora_b_t, int64_t rank, float scaling,
                int64_t rows, int64_t in_features, int64_t out_features, void* grad_x, int64_t ld_grad_x,
                float* grad_a, float* grad_b, void* workspace, int64_t workspace_bytes, int dtype,
                void* stream);

/* ------------------------------------------------------------------------
 * Boundary adjoints
 * ---------------------------------------------------------------------- */

/* Reduction of the consumer adjoints of a shared forest segment into its
 * parent adjoint: replaces the fused reduction of
 * engine/boundary_adjoint.py:49-115 (_boundary_adjoint_reduce_kernel, called
 * by _triton_reduce, :201-225).  out = cast(existing + adjoints[0] + ... +
 * adjoints[n - 1]), summed in fp32 in that order (without existing: from 0)
 * and cast once to dtype.  adjoints: host array of n_adjoints (0..16) device
 * pointers, each n_elements of dtype; existing: device pointer or NULL (at
 * least one input); every pointer 16-byte aligned; out must not alias an
 * input; with n_elements == 0 nothing is accessed.  Inputs are not modified. */
int ts_adjoint_reduce(const void* const* adjoints, int n_adjoints, const void* existing, void* out,
                      int64_t n_elements, int dtype, void* stream);

/* FP32 adjoint ledger (engine/streaming.py:2647-2665, _ledger_accumulate):
 * init != 0: ledger = widen(contribution) (the first contribution's widening
 * copy); init == 0: ledger += widen(contribution) (the mixed-dtype add_).
 * ledger: n_elements fp32; contribution: n_elements of dtype; both 16-byte
 * aligned and distinct. */
int ts_ledger_add(float* ledger, const void* contribution, int64_t n_elements, int dtype, int init,
                  void* stream);

/* ------------------------------------------------------------------------
 * Forest metadata (host code: every pointer below is host memory)
 * ------------------------------------------------------------------------ */

/* The exact shared forest of a batch of trajectories: replaces build_forest
 * (engine/segments.py:280-346) and its shared-prefix partition (:243-278).
 * Trajectory i's keys (2 * token + scored) are keys[key_offsets[i] ..
 * key_offsets[i + 1]) (at least one each) and its group is group_id[i].
 * Nodes come out numbered in pre-order (groups ascending, children by
 * ascending first key): node n holds keys[key_offsets[node_src[n]] +
 * node_offset[n] ..] of length node_len[n] (0 only for a root), its parent
 * (-1 for a root), depth and group; leaf_of[i] is trajectory i's last node.
 * Node arrays hold max_nodes >= 2 * n_traj entries. */
int ts_forest_build(int64_t n_traj, const int64_t* group_id, const int64_t* key_offsets, const int64_t* keys,
                    int64_t max_nodes, int64_t* n_nodes, int64_t* node_parent, int64_t* node_depth,
                    int64_t* node_group, int64_t* node_src, int64_t* node_offset, int64_t* node_len,
                    int64_t* leaf_of);

/* The execution plan of a forest: replaces compile_plan
 * (engine/plan.py:166-340).  order: the nodes in DFS pre-order (parents
 * first); node n's keys are keys[node_key_offsets[n] .. + node_len[n]);
 * traj_leaf / traj_id: each trajectory's leaf node and id, in the forest's
 * trajectory order.  Outputs: token_ids, position_ids, node_of and
 * subtree_end of P = sum(node_len) physical rows; node_start / node_end per
 * node; score_src / score_tgt / score_pos of *n_scored <= P slots;
 * logical_to_slot / logical_traj of *n_logical <= max_logical entries. */
int ts_plan_compile(int64_t n_nodes, const int64_t* node_parent, const int64_t* order, const int64_t* node_len,
                    const int64_t* node_key_offsets, const int64_t* keys, int64_t n_traj, const int64_t* traj_leaf,
                    const int64_t* traj_id, int64_t max_logical, int64_t* token_ids, int64_t* position_ids,
                    int64_t* node_of, int64_t* node_start, int64_t* node_end, int64_t* subtree_end,
                    int64_t* score_src, int64_t* score_tgt, int64_t* score_pos, int64_t* n_scored,
                    int64_t* logical_to_slot, int64_t* logical_traj, int64_t* n_logical);

/* ------------------------------------------------------------------------
 * Diagnostics
 * ------------------------------------------------------------------------ */

/* Per-kernel device timing.  While enabled, every kernel launch of the
 * library is bracketed by two HIP events recorded on its own stream;
 * ts_timing_read sums the elapsed milliseconds of the bracketed launches of
 * one kernel ("attention.fwd_kernel", "logprob.dlogits_kernel", ...) and
 * ts_timing_reset forgets them.  No counterpart in the reference (its
 * timing goes through torch.profiler / CUDA events around whole
 * operators, grpo/reward_linear.py:95-105); used by bench.py to report
 * each kernel's achieved rate against its roofline. */
int ts_timing_enable(int enable);
int ts_timing_reset(void);
int ts_timing_read(const char* kernel, double* total_ms, int64_t* launches);

/* The device's compute-unit count, peak engine clock (kHz), memory clock
 * (kHz) and memory bus width (bits), from hipDeviceGetAttribute.  bench.py
 * derives its MFMA peak from the first two.  No counterpart in the
 * reference. */
int ts_device_clocks(int device, int* cus, int* clock_khz, int* mem_clock_khz, int* mem_bus_bits);


#ifdef __cplusplus
}
#endif

#endif /* THUNDERSYNC_HIP_H */
