/*
 * cqgdn - C ABI of the MI355X (gfx950) gated delta-rule (GDN) backend.
 *
 * This is the drop-in boundary of the `gdn_backend: hip` path.  It replaces the
 * device ops that the reference binds in ops/gated_delta_net.py (AscendC
 * `fla_npu` ops plus FLA Triton helpers, ops/gated_delta_net.py:24-57).  All
 * pointers are device pointers unless stated; tensors are dense row-major with
 * the layouts given per function; `stream` is a hipStream_t (NULL = default
 * stream).  Every call only enqueues work on `stream` and never synchronizes.
 * Functions return CQGDN_OK or an error code; cqgdn_last_error() gives the
 * message of the last failure on the calling thread.
 *
 * Layouts (T = events, H = heads, D = 128 head dimension):
 *   q, k, v, o, dq, dk, dv, do : bf16 [T][H][D]   (the reference's TND order, B = 1);
 *                                fp16 with CQGDN_FP16
 *   g, beta, dg, dbeta         : fp32 [T][H]
 *   chunk_table                : int32 [n_chunks][2] = (first event, length <= 64);
 *                                chunks never cross a document boundary
 *   doc_chunk                  : int32 [n_docs + 1], chunks of document d are
 *                                doc_chunk[d] .. doc_chunk[d+1]-1, in time order
 *   states                     : fp32 [n_docs][H][K=128][V=128] (key-first), as the
 *                                reference's prefill returns them (ops/gated_delta_net.py:297-311)
 */
#ifndef CQGDN_H_
#define CQGDN_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CQGDN_OK 0
#define CQGDN_EINVAL 1       /* contract violation (shape, null pointer, size) */
#define CQGDN_EUNSUPPORTED 2 /* valid request this build does not implement   */
#define CQGDN_EHIP 3         /* a HIP runtime call failed                      */

#define CQGDN_HEAD_DIM 128
#define CQGDN_CHUNK 64

/* flags of cqgdn_fwd / cqgdn_bwd */
#define CQGDN_NORMALIZE 1u /* l2-normalize q and k in the kernels (use_qk_l2norm_in_kernel=True) */
#define CQGDN_TRAINING 2u  /* the workspace will feed cqgdn_bwd (excludes CQGDN_PRECISE) */
/* Inference forward with fp16 MFMA operands (11-bit mantissa instead of bf16's 8) for final
 * states within 1e-3 of an fp32 computation; V and the initial state are scaled by a power of
 * two inside the call so every fp16 operand stays in range.  Not combinable with CQGDN_TRAINING. */
#define CQGDN_PRECISE 4u
/* With CQGDN_TRAINING: rebuild only the workspace cqgdn_bwd reads, without the output kernel (o is
 * not written and may be NULL).  The backward's recompute of the reference's `fused` mode, which
 * keeps no w / h / v_new between the forward and the backward (ops/gated_delta_net.py:143-156,192-194). */
#define CQGDN_NO_OUTPUT 8u
/* q, k, v and o (cqgdn_fwd), and dout, dq, dk, dv (cqgdn_bwd, cqgdn_bwd_recompute) are fp16
 * [T][H][D] instead of bf16, and every kernel computes with fp16 MFMA operands (as CQGDN_PRECISE
 * does for bf16 inputs): the reference's fp16 training and prefill (ops/gated_delta_net.py:233-234).
 * V, the initial state and (in the backward) dout are scaled by powers of two inside the calls so
 * that the fp16 operands stay in range.  Combinable with CQGDN_TRAINING; a cqgdn_bwd call passes it
 * exactly when the cqgdn_fwd call that made its workspace did. */
#define CQGDN_FP16 16u

/* Library version string, e.g. "cqgdn 0.1.0 gfx950". */
const char* cqgdn_version(void);

/* Message of the last error returned on this thread ("" if none). */
const char* cqgdn_last_error(void);

/*
 * Host helper: chunk table of packed documents.  bounds (host int64,
 * n_bounds entries) are cumulative document boundaries (0, ..., T) as checked by
 * host_bounds() (ops/gated_delta_net.py:102-114).  Replaces chunk_indices()
 * (ops/gated_delta_net.py:90-99) for chunk size 64.  With table == NULL only the
 * counts are returned.  Returns the number of chunks, or -1 on invalid bounds.
 */
int64_t cqgdn_chunk_table(const int64_t* bounds, int n_bounds, int32_t* table, int32_t* doc_chunk);

/*
 * Forward workspace: size in bytes, and the byte offset of each of its
 * CQGDN_FWD_BUFFERS internal buffers (order documented in gdn_layout.hpp) so
 * that tests can inspect intermediates.  The same workspace must be passed,
 * unmodified, to cqgdn_bwd, with the same q and k (the workspace keeps the
 * per-row l2 scales of k, not normalized copies; the kernels that read q form
 * its scales themselves).
 */
#define CQGDN_FWD_BUFFERS 9
#define CQGDN_BWD_BUFFERS 8
size_t cqgdn_fwd_workspace_size(int64_t T, int H, int64_t n_chunks);
int cqgdn_fwd_buffer_offsets(int64_t T, int H, int64_t n_chunks, size_t* offsets, int count);
size_t cqgdn_bwd_workspace_size(int64_t T, int H, int64_t n_chunks);
int cqgdn_bwd_buffer_offsets(int64_t T, int H, int64_t n_chunks, size_t* offsets, int count);

/*
 * Chunked GDN forward (fused l2norm, chunk cumsum, beta*K K^T, UT inverse, w/u,
 * inter-chunk state scan, output).  Replaces `chunk_gated_delta_rule_fwd`
 * (ops/gated_delta_net.py:144-156 training, :297-309 prefill) and the cached
 * chain l2_fwd / chunk_local_cumsum / chunk_scaled_dot_kkt / solve_tril /
 * recompute_w_u_fwd / chunk_gated_delta_rule_fwd_h / chunk_fwd_o
 * (ops/gated_delta_net.py:136-137,158-183).
 *   scale          : output scale (the reference uses D^-0.5, ops/gated_delta_net.py:248)
 *   initial_state  : NULL or [n_docs][H][K][V] fp32 starting state per document
 *   final_state    : NULL or [n_docs][H][K][V] fp32, written with each document's last state
 *   o              : [T][H][D] output (time-first), bf16 (fp16 with CQGDN_FP16)
 *   workspace      : >= cqgdn_fwd_workspace_size() bytes, 256-byte aligned
 *   flags          : CQGDN_NORMALIZE | (CQGDN_TRAINING or CQGDN_PRECISE) | CQGDN_FP16 with fp16
 *                    q/k/v/o; the reference's prefill (ops/gated_delta_net.py:292-311) maps to
 *                    NORMALIZE | PRECISE (| FP16 for fp16 inputs).
 *                    A CQGDN_TRAINING forward takes no initial_state and no final_state.
 */
int cqgdn_fwd(const void* q, const void* k, const void* v, const float* g, const float* beta, int64_t T, int H,
              const int32_t* chunk_table, int64_t n_chunks, const int32_t* doc_chunk, int n_docs, float scale,
              unsigned flags, const float* initial_state, float* final_state, void* o, void* workspace,
              size_t workspace_bytes, void* stream);

/*
 * cqgdn_fwd for callers that cannot allocate device memory (code under HIP graph
 * capture, serving loops, harnesses that forbid hipMalloc).  No counterpart in the
 * reference.  The same forward, with the same arguments minus the workspace: it
 * uses the library's own static workspace of CQGDN_STATIC_WORKSPACE_BYTES per GPU
 * (a file-scope device array, held until the process ends) and calls no allocator.
 * It rejects with CQGDN_EINVAL any call whose cqgdn_fwd_workspace_size exceeds that
 * (at H = 16 and one document: up to 2,496 events), and CQGDN_TRAINING (the workspace does not
 * outlive the call, so it cannot feed cqgdn_bwd).  Every call on one GPU shares
 * that GPU's workspace, which keeps the last call's contents: calls that overlap
 * on one GPU (two streams, or two threads) race and must be serialized by the
 * caller.  Nothing in the workspace needs to start at zero.
 *
 * The array is reserved when the runtime loads the code object that holds it, which
 * happens at its first address lookup on a device: call cqgdn_fwd_static_init() once
 * per device at set-up (with that device current) so that no cqgdn_fwd_static call
 * reserves memory; without it, the first cqgdn_fwd_static call on a device does the
 * lookup.  Processes that never call either reserve nothing.
 */
#define CQGDN_STATIC_WORKSPACE_BYTES (64u << 20)
int cqgdn_fwd_static(const void* q, const void* k, const void* v, const float* g, const float* beta, int64_t T,
                     int H, const int32_t* chunk_table, int64_t n_chunks, const int32_t* doc_chunk, int n_docs,
                     float scale, unsigned flags, const float* initial_state, float* final_state, void* o,
                     void* stream);

/* Set-up of cqgdn_fwd_static on the current device (no counterpart in the reference; for the
 * same callers): looks up the device's static workspace once, reserving its
 * CQGDN_STATIC_WORKSPACE_BYTES, and keeps its address for later calls.  Idempotent. */
int cqgdn_fwd_static_init(void);

/*
 * Chunked GDN backward from the forward workspace (which must come from a
 * cqgdn_fwd call with CQGDN_TRAINING on the same inputs).  Replaces the
 * backward op chain of _Delta.backward (ops/gated_delta_net.py:188-214:
 * chunk_bwd_dv_local, chunk_gated_delta_rule_bwd_dhu, chunk_bwd_dqkwg,
 * prepare_wy_repr_bwd_da, prepare_wy_repr_bwd_full, reverse_cumsum, l2_bwd).
 * The reference keeps the normalized q, k and their rstd (ctx.save_for_backward,
 * :184); this call takes the inputs q, k and forms the normalized rows from the
 * rstd kept in the workspace, rounded as the forward rounded them.  Gradients are
 * written in the input layouts: dq, dk, dv bf16 [T][H][D] (fp16 with CQGDN_FP16, which
 * must match the forward's flags); dg, dbeta fp32 [T][H].
 */
int cqgdn_bwd(const void* q, const void* k, const void* v, const float* g, const float* beta, const void* dout,
              int64_t T, int H, const int32_t* chunk_table, int64_t n_chunks, const int32_t* doc_chunk, int n_docs,
              float scale, unsigned flags, const void* fwd_workspace, size_t fwd_workspace_bytes,
              void* bwd_workspace, size_t bwd_workspace_bytes, void* dq, void* dk, void* dv, float* dg, float* dbeta,
              void* stream);

/*
 * The backward of the reference's `fused` mode in one call: the forward workspace is
 * rebuilt from q, k, v, g, beta (cqgdn_fwd with CQGDN_TRAINING | CQGDN_NO_OUTPUT) and
 * then consumed by the backward (cqgdn_bwd).  Replaces _Delta.backward when no w / h / v_new
 * were kept (ops/gated_delta_net.py:188-194: recompute_w_u_fwd and
 * chunk_gated_delta_rule_fwd_h, then the chain of :195-214).  Arguments as cqgdn_fwd and
 * cqgdn_bwd; fwd_workspace is written here and needs no contents on entry.
 * The rebuilt forward state scan runs on a second stream beside the backward's local
 * kernel and reverse scan (neither reads h or v_new; each scan holds half of the CUs),
 * and the last backward kernel waits for it.  That stream and its two events are
 * created on a thread's first call on a device and kept until the process ends; the
 * call orders them against `stream` with events, so it can be captured in a HIP graph.
 */
int cqgdn_bwd_recompute(const void* q, const void* k, const void* v, const float* g, const float* beta,
                        const void* dout, int64_t T, int H, const int32_t* chunk_table, int64_t n_chunks,
                        const int32_t* doc_chunk, int n_docs, float scale, unsigned flags, void* fwd_workspace,
                        size_t fwd_workspace_bytes, void* bwd_workspace, size_t bwd_workspace_bytes, void* dq,
                        void* dk, void* dv, float* dg, float* dbeta, void* stream);

/*
 * Recurrent GDN step(s): for each of N independent sequences, E events applied
 * in order to a value-first fp32 state [N][H][V][K], updated in place, as the
 * decode path does with the FLA kernel fused_recurrent_gated_delta_rule_fwd_kernel
 * (ops/gated_delta_net.py:314-352; math of models/decoding.py:71-77):
 *   S <- exp(g) S ; S <- S + beta k (v - S k)^T ; o = scale S q
 * q, k (already l2-normalized), v, out: [N][E][H][D], bf16 (or fp16 with
 * CQGDN_RECURRENT_FP16); g: fp32 [N][E][H]; beta: [N][E][H], fp32 (or bf16 with
 * CQGDN_RECURRENT_BETA_BF16).  dtype_flags 0 and 1 keep their meaning of the
 * former beta_is_bf16 argument.  The reference call is N = 1.
 */
#define CQGDN_RECURRENT_BETA_BF16 1
#define CQGDN_RECURRENT_FP16 2
int cqgdn_recurrent(const void* q, const void* k, const void* v, const float* g, const void* beta, int dtype_flags,
                    float* state, void* out, int N, int E, int H, float scale, void* stream);

/*
 * Row-wise l2norm over D = 128 (the `l2_fwd` / `l2_bwd` ops bound at
 * ops/gated_delta_net.py:52-53 and used at :136-137, :207-209 and
 * models/decoding.py:63-64): y = x * rsqrt(sum x^2 + 1e-6), rstd optional.
 * Backward: dx = rstd * (dy - y (y . dy)).  x, y, dy, dx: bf16 [rows][128].
 */
int cqgdn_l2norm_fwd(const void* x, void* y, float* rstd, int64_t rows, void* stream);
int cqgdn_l2norm_bwd(const void* y, const float* rstd, const void* dy, void* dx, int64_t rows, void* stream);

/*
 * Packed depthwise causal conv1d (the GatedDelta layer's short conv over the
 * q/k/v channels).  Replaces the causal_conv1d_fn / causal_conv1d_bwd calls of
 * conv() (ops/gated_delta_net.py:252-289); semantics of the CPU form
 * F.conv1d(padding = K - 1) per document (models/backbone_qwen35.py:81-98):
 *   pre[t][c] = sum_{i<K} w[c][i] * x[t - (K-1) + i][c] over rows of t's document,
 *   y = silu(pre) if activation != 0, else pre.
 * x, y, dy, dx: bf16 [T][C], time-first (B = 1), C % 8 == 0, 16-byte aligned;
 * weight: bf16 [C][K], 2 <= K <= 4; bounds: device int32 [n_docs + 1] document
 * boundaries (0, ..., T).  The backward recomputes pre from x (nothing is saved
 * by the forward) and writes dweight fp32 [C][K] through a deterministic
 * reduction of per-row-strip partials held in the workspace
 * (>= cqgdn_conv1d_bwd_workspace_size bytes, 16-byte aligned).
 */
int cqgdn_conv1d_fwd(const void* x, const void* weight, const int32_t* bounds, int n_docs, int64_t T, int C, int K,
                     int activation, void* y, void* stream);
size_t cqgdn_conv1d_bwd_workspace_size(int64_t T, int C, int K);
int cqgdn_conv1d_bwd(const void* x, const void* weight, const void* dy, const int32_t* bounds, int n_docs, int64_t T,
                     int C, int K, int activation, void* dx, float* dweight, void* workspace, size_t workspace_bytes,
                     void* stream);

/*
 * Gated RMSNorm over D = 128 fused with the layer's output gather.  Replaces
 * gated_norm() (ops/gated_delta_net.py:67-74; CPU form GatedNorm.forward,
 * models/backbone_qwen35.py:107-114) applied to y.index_select(0, hidden_event)
 * with the padding rows zeroed (models/backbone_qwen35.py:242-246):
 *   x = index ? (index[r] >= 0 ? y[index[r]][h] : 0) : y[r][h]
 *   out[r][h] = x * rsqrt(mean(x^2) + eps) * weight * silu(z[r][h])
 * y: bf16 [y_rows][H][128]; index: NULL or device int32 [rows], each value in
 * [-1, y_rows) (-1: a padding row); z: bf16 rows of H*128 channels, z_stride
 * elements apart (a column slice of the layer's fused projection is accepted);
 * weight: fp32 [128]; out: bf16 [rows][H][128]; rstd: fp32 [rows][H], kept for
 * the backward.  Computed in fp32 with one rounding of out.
 */
int cqgdn_gated_norm_fwd(const void* y, const int32_t* index, int64_t rows, int H, const void* z, int64_t z_stride,
                         const float* weight, float eps, void* out, float* rstd, void* stream);
/*
 * Backward of cqgdn_gated_norm_fwd.  Row index[r] of dy bf16 [y_rows][H][128]
 * receives row r's gradient (index must not repeat a value >= 0), and each of
 * the n_zero rows listed in zero_rows (device int32: the y rows no r reads) is
 * written with zeros, so that every dy row is written once and no atomics are
 * needed; without index, dy row r is row r's gradient.  dz: bf16 rows at
 * dz_stride elements; dweight: fp32 [128] through a deterministic reduction of
 * per-workgroup partials held in the workspace (>= the size below, 16-byte
 * aligned).
 */
size_t cqgdn_gated_norm_bwd_workspace_size(int64_t rows, int H);
int cqgdn_gated_norm_bwd(const void* y, const int32_t* index, const int32_t* zero_rows, int64_t n_zero, int64_t rows,
                         int H, const void* z, int64_t z_stride, const float* weight, const float* rstd,
                         const void* dout, void* dy, void* dz, int64_t dz_stride, float* dweight, void* workspace,
                         size_t workspace_bytes, void* stream);

/*
 * One layer's event plan as device int32 arrays: the DeltaPlan fields the
 * GatedDelta layer reads (ops/gated_delta_layout.py:13-27, built at :54-176),
 * plus inverse maps the host derives once per plan.  Content rows are
 * 0 .. n_content-1; the value n_content stands for "none" / the zero row, as in
 * the reference's torch.cat((x, zeros)).index_select idiom.
 */
typedef struct cqgdn_event_plan {
  int32_t n_content, n_queries, n_events, conv_kernel; /* conv_kernel K: 2..4 */
  const int32_t* content_order;  /* [n_content] hidden row of each content write (plan.content_order) */
  const int32_t* event_q;        /* [n_events] q source: content row, or n_content + query (plan.event_q) */
  const int32_t* event_write;    /* [n_events] content row written, n_content if read-only (plan.event_write) */
  const int32_t* query_source;   /* [n_queries] hidden row of each query (plan.query_source) */
  const int32_t* query_history;  /* [n_queries][K-1] content rows of each query's conv history */
  const int32_t* content_bounds; /* [n_content_docs + 1] document bounds of the content conv */
  int32_t n_content_docs;
  int32_t n_history_rows;        /* entries of history_rows */
  const int32_t* q_ptr;          /* [n_content + 1] CSR: the events whose q is content row c ... */
  const int32_t* q_list;         /*   ... in event order */
  const int32_t* write_event;    /* [n_content] the event writing content row c, -1 if none */
  const int32_t* query_event;    /* [n_queries] the event reading query j */
  const int32_t* history_ptr;    /* [n_content + 1] CSR: j * (K-1) + i with query_history[j][i] == c ... */
  const int32_t* history_list;   /*   ... ascending */
  const int32_t* history_rows;   /* content rows with at least one history entry */
  /* Content rows sharing a hidden row: the reference's Bi_I+CQ_T plans re-write the
   * generation prefix's hidden rows in a second branch (ops/gated_delta_layout.py:66-83),
   * so content_order repeats them.  n_fold_rows = 0 when content_order repeats no row;
   * otherwise the distinct hidden rows of content_order, with a CSR of the content rows
   * reading each, over which the backward sums their gradients (fixed order). */
  int32_t n_fold_rows;
  const int32_t* fold_rows;      /* [n_fold_rows] distinct hidden rows of content_order */
  const int32_t* fold_ptr;       /* [n_fold_rows + 1] CSR: the content rows reading fold_rows[i] ... */
  const int32_t* fold_list;      /*   ... ascending */
} cqgdn_event_plan;

/*
 * The recurrence's event inputs from the layer's projection, in two launches:
 * the packed causal conv (with SiLU) over the content rows, read from the
 * projection through content_order; then per event q (a content row of the conv
 * output, or a CQ query whose conv reads its own row and its history rows), k
 * and v (the written content row, or zeros), g = -exp(A_log) softplus(a +
 * dt_bias) and beta = sigmoid(b) (zeros for read-only events).  Replaces
 * models/backbone_qwen35.py:166-194 (index_select, conv1d, the query conv, the
 * cat/index_select gathers and the gate math).
 *   H value heads and key_heads key heads (both 4, 8, 16 or 32, key_heads
 *   dividing H; the reference's linear_value_heads and linear_heads per rank):
 *   value head j reads key head j / (H / key_heads), as the reference's
 *   repeat_interleave (models/backbone_qwen35.py:182-183), so q and k come out
 *   with H heads like v;
 *   raw: bf16 rows of C = SK + SK + SV channels (q | k | v, SK = key_heads * 128,
 *   SV = H * 128) raw_stride apart; a, b: bf16 rows of H gate inputs, a_stride /
 *   b_stride apart (all three may be column slices of the fused projection);
 *   conv_weight: bf16 [C][K]; A_log, dt_bias: fp32 [H]; q, k, v: bf16
 *   [n_events][H][128]; g, beta: fp32 [n_events][H]; workspace: >=
 *   cqgdn_event_inputs_fwd_workspace_size bytes.
 */
size_t cqgdn_event_inputs_fwd_workspace_size(int n_content, int H, int key_heads);
int cqgdn_event_inputs_fwd(const cqgdn_event_plan* plan, int H, int key_heads, const void* raw, int64_t raw_stride,
                           const void* a, int64_t a_stride, const void* b, int64_t b_stride, const void* conv_weight,
                           const float* A_log, const float* dt_bias, void* q, void* k, void* v, float* g, float* beta,
                           void* workspace, size_t workspace_bytes, void* stream);
/*
 * Backward of cqgdn_event_inputs_fwd from the recurrence's gradients dq, dk, dv
 * (bf16 [n_events][H][128]) and dg, dbeta (fp32 [n_events][H]).  Writes the
 * raw, a and b gradient rows of every content and query row (d_raw, d_a, d_b,
 * same layouts as raw, a, b; other rows are not touched), dweight fp32 [C][K]
 * and dgate fp32 [2H] (A_log, then dt_bias).  A key head's q and k gradients
 * are the sums over its value heads.  The scatters walk the plan's
 * inverse maps, so every output is written once, without atomics, and the
 * result is deterministic.  A hidden row read by several content rows
 * (n_fold_rows > 0) receives the sum of their gradients.  The workspace size
 * depends on the plan (it holds per-content-row gradients when rows are shared).
 */
size_t cqgdn_event_inputs_bwd_workspace_size(const cqgdn_event_plan* plan, int H, int key_heads);
int cqgdn_event_inputs_bwd(const cqgdn_event_plan* plan, int H, int key_heads, const void* raw, int64_t raw_stride,
                           const void* a, int64_t a_stride, const void* b, int64_t b_stride, const void* conv_weight,
                           const float* A_log, const float* dt_bias, const void* dq, const void* dk, const void* dv,
                           const float* dg, const float* dbeta, void* d_raw, int64_t d_raw_stride, void* d_a,
                           int64_t d_a_stride, void* d_b, int64_t d_b_stride, float* dweight, float* dgate,
                           void* workspace, size_t workspace_bytes, void* stream);

/*
 * One decode step of the GatedDelta layer for N independent sequences, each
 * advancing by one sampled content token C and one text-mask query Q.  Replaces
 * delta_step (models/decoding.py:16-78) between the layer's projection and
 * out_proj, in one launch with one workgroup per (sequence, value head): the conv step
 * of C over the conv history (which then shifts in C's raw row) and Q's query
 * conv over the updated history, the l2 norms and gates; the recurrence over
 * the two events (Q read-only); the gated norm with z from the projection rows.
 * It needs no workspace: cqgdn_layer_decode_workspace_size returns 0 and
 * workspace may be NULL (both stay in the signature so that callers keep working).
 *   Heads and channels as in cqgdn_event_inputs_fwd (with fewer key heads than
 *   value heads a second, small launch shifts the key heads' conv history);
 *   proj: bf16 [N][2][proj_stride] (row 0 = C, row 1 = Q; columns q|k|v, z, a, b
 *   of the fused projection); conv_history: bf16 [N][K-1][C], updated in place;
 *   conv_weight: bf16 [C][K]; A_log, dt_bias: fp32 [H]; norm_weight: fp32 [128];
 *   scale: the q scale (the reference uses 128^-0.5); state: fp32 [N][H][V][K]
 *   value-first (as cqgdn_recurrent), updated in place; out: bf16 [N][2][H][128].
 */
size_t cqgdn_layer_decode_workspace_size(int N, int H);
int cqgdn_layer_decode_step(int N, int H, int key_heads, int conv_kernel, const void* proj, int64_t proj_stride,
                            void* conv_history, const void* conv_weight, const float* A_log, const float* dt_bias,
                            const float* norm_weight, float eps, float scale, float* state, void* out, void* workspace,
                            size_t workspace_bytes, void* stream);

/*
 * Chunk-local cumsum of g fp32 [T][H] over the chunk table, forward or reverse
 * (`chunk_local_cumsum` and reverse_cumsum(), ops/gated_delta_net.py:77-87,158-164).
 */
int cqgdn_chunk_local_cumsum(const float* g, float* out, int64_t T, int H, const int32_t* chunk_table,
                             int64_t n_chunks, int reverse, void* stream);

/*
 * Instrumentation (no counterpart in the reference; used by the benchmark to
 * price one kernel against its roofline).  cqgdn_timer_arm(name, n) makes the
 * library bracket each of the next n launches of the named kernel with
 * hipEventRecord on the stream it is launched on; name = NULL disarms.  Names:
 * fwd_prep, fwd_scan, fwd_out, bwd_local, bwd_scan, bwd_dkw,
 * recurrent.  cqgdn_timer_read waits for the recorded
 * events, writes up to `capacity` per-launch durations in milliseconds,
 * stores the number of launches recorded, and disarms.  One kernel is armed
 * at a time, process-wide.  Both return CQGDN_OK, CQGDN_EINVAL (unknown name
 * or n outside 1..65536) or CQGDN_EHIP; they do not set cqgdn_last_error().
 */
int cqgdn_timer_arm(const char* kernel, int max_launches);
int cqgdn_timer_read(float* launch_ms, int capacity, int* launches);

#ifdef __cplusplus
}
#endif

#endif /* CQGDN_H_ */
