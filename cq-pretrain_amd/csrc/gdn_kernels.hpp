// Host-side argument blocks and launchers of the GDN kernels (internal to libcqgdn).
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "gdn_layout.hpp"
#include "gdn_timer.hpp"

namespace cqgdn {

typedef __bf16 bf16;

struct FwdArgs {
  const void *q, *k, *v;     // bf16, or fp16 with fp16 (both [T][H][D])
  const float *g, *beta;
  const int32_t* chunks;     // [n_chunks][2] (start, len)
  const int32_t* doc_chunk;  // [n_docs + 1]
  int T, H, n_chunks, n_docs;
  float scale;
  bool normalize;
  bool precise;                // fp16 operands from bf16 inputs (inference); the workspace then holds fp16
  bool fp16;                   // fp16 inputs and output, fp16 operands (inference or training)
  bool training;               // the workspace feeds the backward (V's scale target, with fp16 operands)
  bool no_output;              // rebuild the workspace only (the backward's recompute): no output kernel
  const float* initial_state;  // [n_docs][H][K][V] or null
  float* final_state;          // [n_docs][H][K][V] or null
  void* o;                     // [T][H][D], in the inputs' type
  uint8_t* ws;
  size_t off[F_COUNT];
  // optional: the state scan runs on scan_stream, after scan_fork (recorded on the
  // caller's stream behind fwd_prep); scan_join is recorded behind it
  hipStream_t scan_stream;
  hipEvent_t scan_fork, scan_join;
};

struct BwdArgs {
  const void *q, *k, *v, *dout;  // bf16, or fp16 with fp16 (as dq, dk, dv)
  const float *g, *beta;
  const int32_t* chunks;
  const int32_t* doc_chunk;
  int T, H, n_chunks, n_docs;
  float scale;
  bool normalize;
  bool fp16;           // fp16 inputs and gradients, fp16 operands (the forward workspace's too)
  const uint8_t* fws;  // forward workspace
  size_t foff[F_COUNT];
  uint8_t* bws;        // backward workspace
  size_t boff[B_COUNT];
  void *dq, *dk, *dv;
  float *dg, *dbeta;
  hipEvent_t dkw_after;  // optional: bwd_dkw waits for this event (the forward scan's join)
  // optional: bwd_dkw runs on `side` beside the reverse scan (after side_fork, recorded
  // on the caller's stream behind bwd_local; side_join is recorded behind it)
  hipStream_t side;
  hipEvent_t side_fork, side_join;
  // failure-handling tests only: bwd_dkw beside the scan waits for a count the scan
  // never reaches, with a short poll limit, so every chunk's wait gives up
  bool dkw_never_ready;
};

// Both return the first error of their stream-ordering calls (hipSuccess without them);
// launch errors are left for hipGetLastError.
hipError_t launch_fwd(const FwdArgs& a, hipStream_t stream);
hipError_t launch_bwd(const BwdArgs& a, hipStream_t stream);
// out[1 .. kVscaleBlocks] = partial maxima of |x| over n8 groups of 8 values of x (bf16,
// or fp16) and ns fp32 values of s0; the first kernel that needs the power-of-two scale
// forms it from them (range_scale in gdn_common.hpp) and stores it in out[0] (gdn_fwd.hip)
void launch_range_partials(const void* x, bool fp16, size_t n8, const float* s0, size_t ns, float* out,
                           hipStream_t stream);

void launch_recurrent(const void* q, const void* k, const void* v, const float* g, const void* beta,
                      bool beta_bf16, bool fp16, float* state, void* out, int N, int E, int H, float scale,
                      hipStream_t stream);
// packed depthwise causal conv1d (gdn_conv.hip); bounds: int32 [n_docs + 1] on the device
int conv_strips(int64_t T);  // row strips of the conv backward (dw partials per strip)
// x row u is x + (xrows ? xrows[u] : u) * xs; dx row t is dx + (dxrows ? dxrows[t] : t) * dxs; y and dy are [T][C]
void launch_conv_fwd(const bf16* x, const int32_t* xrows, int64_t xs, const bf16* w, const int32_t* bounds,
                     int n_docs, int T, int C, int K, int act, bf16* y, hipStream_t stream);
void launch_conv_bwd(const bf16* x, const int32_t* xrows, int64_t xs, const bf16* w, const bf16* dy,
                     const int32_t* bounds, int n_docs, int T, int C, int K, int act, bf16* dx, const int32_t* dxrows,
                     int64_t dxs, float* dw, float* part, hipStream_t stream);
// out[j] = sum over p < parts of part[p][j], fixed order (gdn_conv.hip); n % 4 == 0, 16-byte aligned part
void launch_colsum(const float* part, int parts, int n, float* out, hipStream_t stream);
// Event inputs of one GatedDelta layer (gdn_glue.hip).  S = H * 128 channels per
// q/k/v part; index arrays are device int32 (content rows are 0 .. n_c-1, n_c is
// the zero row / "none").
// Heads: H value heads and HK key heads, G = H / HK = 1 << gshift value heads per
// key head (value head j reads key head j >> gshift, as the reference's
// repeat_interleave(h // hk) does).  Projection and conv channels are
// q [0, SK) | k [SK, 2 SK) | v [2 SK, 2 SK + SV), SK = HK * 128, SV = H * 128.
constexpr int EV_MAX_GROUP = 8;  // H / HK with both in {4, 8, 16, 32}
struct EvArgs {
  int H, HK, gshift, K, n_c, n_q, E, n_hrows;
  const int32_t* order;    // [n_c] hidden row of content row c
  const int32_t* eq;       // [E] q source: content row, or n_c + query
  const int32_t* ew;       // [E] content row written, n_c for read-only events
  const int32_t* qsource;  // [n_q] hidden row of query j
  const int32_t* qhist;    // [n_q][K-1] content rows of query j's conv history
  const int32_t* qptr;     // [n_c + 1] CSR: events whose q is content row c ...
  const int32_t* qlist;    //   ... in event order
  const int32_t* winv;     // [n_c] event writing content row c, -1 if none
  const int32_t* qev;      // [n_q] event reading query j
  const int32_t* hptr;     // [n_c + 1] CSR: entries j * (K-1) + i with qhist[j][i] == c ...
  const int32_t* hlist;    //   ... ascending
  const int32_t* hrows;    // [n_hrows] content rows with history entries
  const bf16* raw;         // projection rows, channels q | k | v
  int64_t raw_stride;
  const bf16* ga;          // a (H per row)
  int64_t ga_stride;
  const bf16* gb;          // b (H per row)
  int64_t gb_stride;
  const bf16* w;           // conv weight [2 SK + SV][K]
  const float* A_log;      // [H]
  const float* dt_bias;    // [H]
};
struct EvGrads {
  const bf16 *dq, *dk, *dv;  // [E][SV] (value heads)
  const float *dg, *dbeta;   // [E][H]
  bf16* draw;                // gradient rows of raw (every hidden row of order / qsource is written)
  int64_t draw_stride;
  bf16* da;
  int64_t da_stride;
  bf16* db;
  int64_t db_stride;
  float* dw;     // conv weight gradient [2 SK + SV][K]
  float* dgate;  // [2H]: A_log, then dt_bias
  // When content rows share hidden rows (a plan whose content_order repeats a
  // row): the content rows' raw and gate gradients go to these per-content-row
  // buffers instead of the hidden rows, and the fold pass sums them into draw,
  // da, db over the fold CSR.  Null otherwise.
  bf16* dcont;   // [n_c][2 SK + SV]
  float* dcgate; // [n_c][2H]: da, then db
  int n_fold;                 // distinct hidden rows of content_order (when dcont is set)
  const int32_t* fold_rows;   // [n_fold] those hidden rows
  const int32_t* fold_ptr;    // [n_fold + 1] CSR: the content rows reading fold_rows[i] ...
  const int32_t* fold_list;   //   ... ascending
};
struct EvWork {
  bf16* dconv;   // [n_c][2 SK + SV] gradient of the conv output
  float* dpre;   // [n_q][SK] gradient of the query convs' pre-activation
  float* gpart;  // [n_c][2H]
  float* qpart;  // [events_query_blocks][SK][K]
  float* cpart;  // conv backward partials
  float* qsum;   // [SK][K]
};
int events_query_blocks(int n_q);
void launch_events_fwd(const EvArgs& a, const bf16* conv, bf16* q, bf16* k, bf16* v, float* g, float* beta,
                       hipStream_t stream);
void launch_events_bwd(const EvArgs& a, const EvGrads& d, const int32_t* content_bounds, int n_content_docs,
                       const EvWork& w, hipStream_t stream);
// One decode step of the layer (gdn_glue.hip).  proj rows: [N][2][row_stride]
// (C, then Q; columns q|k|v, z, a, b); hist updated in place.
struct DecArgs {
  int N, H, HK, gshift, K;  // heads as in EvArgs
  const bf16* proj;
  int64_t row_stride;
  bf16* hist;     // [N][K-1][2 SK + SV]
  const bf16* w;  // conv weight [2 SK + SV][K]
  const float* A_log;
  const float* dt_bias;
};
// the whole decode step (prep, recurrence, gated norm) in one launch, one workgroup per (sequence, head)
void launch_decode_step(const DecArgs& a, float* state, const float* norm_w, float eps, float scale, bf16* out,
                        hipStream_t stream);
// gated RMSNorm over D = 128 with an optional row gather (gdn_glue.hip)
int gnorm_bwd_blocks(int64_t rows, int H);  // workgroups of the backward (dw partials per workgroup)
void launch_gnorm_fwd(const bf16* y, const int32_t* index, int64_t rows, int H, const bf16* z, int64_t z_stride,
                      const float* w, float eps, bf16* out, float* rstd, hipStream_t stream);
void launch_gnorm_bwd(const bf16* y, const int32_t* index, const int32_t* zero_rows, int64_t n_zero, int64_t rows,
                      int H, const bf16* z, int64_t z_stride, const float* w, const float* rstd, const bf16* dout,
                      bf16* dy, bf16* dz, int64_t dz_stride, float* dw, float* wpart, hipStream_t stream);
void launch_l2norm_fwd(const bf16* x, bf16* y, float* rstd, int64_t rows, hipStream_t stream);
void launch_l2norm_bwd(const bf16* y, const float* rstd, const bf16* dy, bf16* dx, int64_t rows,
                       hipStream_t stream);
// dst[i] = src ? src[i] : 0 (a kernel, not hipMemset, so callers may capture it in a graph)
void launch_copy_or_zero(float* dst, const float* src, size_t n, hipStream_t stream);
void launch_chunk_cumsum(const float* g, float* out, const int32_t* chunks, int n_chunks, int H, bool reverse,
                         hipStream_t stream);

}  // namespace cqgdn
