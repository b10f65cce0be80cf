// GDN backward on gfx950.
//
// Per chunk (C events, S_c the state entering it, dS_{c+1} the gradient of the
// state leaving it), with Gam_ij = exp(G_i - G_j) on i >= j, gam = exp(G),
// kdec_i = exp(G_last - G_i), P = (Qn Kn^T) * Gam:
//
//   bwd_local  (grid NC x H)  dv_local = scale P^T dO ;  X = scale (gam Qn)^T dO
//   bwd_scan   (serial, reverse)  dVn = dv_local + kdec * (Kn dS_{c+1})
//                                 dS_c = exp(G_last) dS_{c+1} + X - W^T dVn
//   bwd_dkw    (grid NC x H), in one workgroup:
//              dQn = scale gam (dO S_c^T) + (scale dP Gam) Kn   (dP = dO Vn^T); l2norm backward of dq
//              dKn(part) = (scale dP Gam)^T Qn + kdec (Vn dS_{c+1}^T)
//              dW = -dVn S_c^T ; dG terms of the output and state update
//              dT = dW (beta gam Kn)^T + dVn (beta V)^T ; dA = -(T^T dT T^T)
//              dKn += beta (dA Gam) Kn + (dA Gam)^T (beta Kn) + beta gam (T^T dW)
//              dV = beta (T^T dVn) ; dbeta ; dG ; reverse cumsum -> dg ; l2norm backward of dk
//
// This is the reference's backward op chain (ops/gated_delta_net.py:188-214:
// chunk_bwd_dv_local, chunk_gated_delta_rule_bwd_dhu, chunk_bwd_dqkwg,
// prepare_wy_repr_bwd_da/_full, reverse_cumsum, l2_bwd) regrouped into three
// kernels.  All reductions run in a fixed order (no atomics), so results are
// bitwise reproducible from run to run.
//
// E is the operand type: bf16, or fp16 for fp16 inputs.  In fp16 every quantity is
// carried in exact power-of-two scales that keep it inside fp16's range: the
// forward's scale s_v of V (h and v_new carry it; the V rows read here are scaled
// by it too) and the scale s_d of dO.  s_d brings max|dO| below 2^e with
// T 2^e <= 2^15: with unit-norm q rows a state gradient satisfies |dS| <= T max|dO|,
// so dS and dVn stay below about 2^15.  dv_local, X, dS, dVn and dv carry s_d; dP,
// dW, dT, dA, dq, dk, dg and dbeta carry s_d s_v.  Each output is divided by its
// scale in fp32 before it is stored.
//
// bwd_dkw may run on a second stream beside the reverse scan (launch_bwd): the
// scan then stores each chunk's dS / dVn at device scope and announces the chunk
// with an atomic count, and bwd_dkw takes the chunks in the order the scan
// finishes them, each waiting (bounded) for its count.  The atomics only order
// the hand-off; every value is computed as in the sequential order, so the
// results are the same bits either way.
#include "gdn_common.hpp"
#include "gdn_layout.hpp"
#include "gdn_kernels.hpp"

namespace cqgdn {

constexpr int LDK = 136;  // bf16 row stride, 64 x 128 tiles
constexpr int LDT = 72;   // bf16 row stride, 128 x 64 and 64 x 64 tiles

// ---------------------------------------------------------------------------
// bwd_local
// ---------------------------------------------------------------------------
// dscale: null in bf16; in fp16 the scale s_d of dO, which this kernel forms from the
// partial maxima after dscale[0] (range_scale, target ds_target) and stores in
// dscale[0] for bwd_dkw
template <class E>
__global__ __launch_bounds__(256, 3) void bwd_local_kernel(
    const E* __restrict__ q, const E* __restrict__ k, int normalize,
    const float* __restrict__ rk, const E* __restrict__ dout, const float* __restrict__ gc,
    const float* __restrict__ beta, const E* __restrict__ Tm,
    const int32_t* __restrict__ chunks, int H, float scale, float* __restrict__ dscale, int ds_target,
    E* __restrict__ dvlT, E* __restrict__ XT, E* __restrict__ knP, E* __restrict__ WT, int* __restrict__ sync) {
  typedef typename Vec<E>::x8 X8;
  constexpr bool F16 = __is_same(E, f16);
  // grid (H, NC), chunks dispatched first to last: the reverse state scan that
  // follows reads the last chunks first, and they are then the most recently
  // written (still in the memory-side cache).  The scan's other two operands,
  // the perm32 copy of Kn and -W^T, are made here for the same reason.
  const HeadChunk hc = xcd_head_chunk(gridDim.x, gridDim.y);  // all heads of a chunk on one XCD
  const int h = hc.h, c = hc.p;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, q4 = lane >> 4;
  const ChunkInfo ci = chunk_info(chunks, c);
  const size_t cb = (size_t)c * H + h;
  // the counts of the reverse scan's hand-off to bwd_dkw start at zero: this (chunk,
  // head)'s, and (one workgroup) the count of resident scan workgroups after them
  if (tid == 0) {
    sync[cb] = 0;
    if (c == 0 && h == 0) sync[(size_t)gridDim.y * H] = 0;
  }

  // Row tiles only (every transposed operand is read with ds_read_b64_tr_b16),
  // 52 KB, so three workgroups share a CU.  The outputs are staged over them
  // once they are read and stored as whole rows: X^T over Qs | Ks, dv_local^T
  // (64-element rows, 16-byte columns XOR-swizzled by row) over dOs.
  __shared__ __attribute__((aligned(16))) E QK[2 * 64 * LDK];  // Qs | Ks, then X^T [v][k]
  __shared__ __attribute__((aligned(16))) E dOs[64 * LDK];     // dO rows, then dv_local^T [v][s]
  __shared__ __attribute__((aligned(16))) float Gs[64];
  __shared__ __attribute__((aligned(16))) float Bs[64];
  __shared__ float red[4];
  E* Qs = QK;
  E* Ks = QK + 64 * LDK;
  static_assert(64 * LDK >= 128 * 64, "dv_local^T fits the dO tile");
  // fp16: this thread's partial maximum of |dO|, requested before the other loads
  const float dpart = F16 ? range_partial4(dscale + 1) : 0.f;
  float ds = 1.f;  // s_d (fp16), formed once the input loads are in flight

  // T rows t = 16 wave + r, for -W^T below (requested with the inputs)
  X8 at[2];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) at[kb] = ld8(Tm + cb * (CH * CH) + (16 * wave + r) * CH + 32 * kb + 8 * q4);
  {
    const int t = tid >> 2, p = tid & 3;
    const bool in = t < ci.len;
    const int tc = clamp_row(t, ci.len);
    const size_t ev = (size_t)(ci.start + tc) * H + h, row = ev * D;
    const float rkt = rk[ev];
    // q and k non-temporally: what this kernel writes (the reverse scan's operands,
    // 188 MB at T = 9216, H = 16) and what the scan writes do not both fit the
    // 256 MB memory-side cache, and q, k are read next only by bwd_dkw, after the scan
    X8 xq[4], xk[4], xd[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int col = 32 * j + 8 * p;
      xq[j] = ld8_nt(q + row + col);
      xk[j] = ld8_nt(k + row + col);
      xd[j] = ld8(dout + row + col);
    }
    if (p == 0) {
      Gs[t] = gc[ev];
      Bs[t] = keep_if(in, beta[ev]);
    }
    const float rqt = normalize ? row_rnorm(xq) : 1.f;
    if constexpr (F16) {  // dO s_d (exact: a power of two, in range)
      ds = range_scale(dpart, ds_target, red);
#pragma unroll
      for (int j = 0; j < 4; ++j) xd[j] = to8<E>(cvtf8(xd[j]) * ds);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int col = 32 * j + 8 * p;
      st8(Qs + t * LDK + col, keep_if(in, scaled8<E>(xq[j], rqt)));
      st8(Ks + t * LDK + col, keep_if(in, scaled8<E>(xk[j], rkt)));
      st8(dOs + t * LDK + col, keep_if(in, xd[j]));
    }
  }
  __syncthreads();

  // perm32 copy of kdec_t Kn_t (kdec_t = exp(G_last - G_t), the decay the
  // reverse scan applies to Kn dS) from the tile: 16-byte piece p of column
  // block j holds logical 32 j + 4 p .. + 3 and 32 j + 16 + 4 p .. + 3
  {
    const int t = tid >> 2, p = tid & 3;
    if (t < ci.len) {
      const float kd = __expf(Gs[ci.len - 1] - Gs[t]);
      E* kp = knP + ((size_t)(ci.start + t) * H + h) * D + 8 * p;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        st8(kp + 32 * j, cat(to4<E>(cvtf4(ld4(Ks + t * LDK + 32 * j + 4 * p)) * kd),
                             to4<E>(cvtf4(ld4(Ks + t * LDK + 32 * j + 16 + 4 * p)) * kd)));
    }
  }

  // per-lane event factors at s = 32 kb + 8 q4 + e: beta_s gam_s (for W) and gam_s (for X)
  f32x8 fbg[2], fg[2];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int s = 32 * kb + 8 * q4 + e;
      fg[kb][e] = __expf(Gs[s]);
      fbg[kb][e] = Bs[s] * fg[kb][e];
    }

  // -W^T [k][perm32(t)] with W = T (beta gam K): t-tile = wave, k-tiles n; beta gam K
  // is read transposed from the K rows and scaled per event s on the way
  {
    E* wt = WT + cb * (D * CH);
#pragma unroll
    for (int n = 0; n < 8; ++n) {
      f32x4 aw = zero4();
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
        if (kb == 0 || wave >= 2)  // T[t][s] = 0 for s > t
          aw = mfma(at[kb], to8<E>(cvtf8(ld8_tr(Ks, LDK, 32 * kb, 16 * n)) * fbg[kb]), aw);
      st4(wt + (16 * n + r) * CH + perm32(16 * wave + 4 * q4), -aw);
    }
  }

  // P tiles (t-tile tt >= s-tile = wave), causal and gated, kept in registers:
  // pp[tt][i] = P[t = 16 tt + 4 q4 + i][s = 16 wave + r]
  f32x4 pp[4];
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
    pp[tt] = zero4();
    if (tt >= wave) {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
        pp[tt] = mfma(ld8(Qs + (16 * tt + r) * LDK + 32 * kb + 8 * q4), ld8(Ks + (16 * wave + r) * LDK + 32 * kb + 8 * q4),
                      pp[tt]);
      const int s = 16 * wave + r;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = 16 * tt + 4 * q4 + i;
        pp[tt][i] = (s <= t) ? pp[tt][i] * __expf(Gs[t] - Gs[s]) : 0.f;
      }
    }
  }

  // dv_local^T (s rows 16 wave + 4 q4 .., 8 value tiles) = P^T dO: P^T comes from
  // the P tiles (pack_perm, events in perm32 order), dO is read transposed in the
  // same order; only t >= s contributes
  f32x4 dvl[8];
  {
    const int kb0 = wave >= 2 ? 1 : 0;
    X8 a[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) a[kb] = pack_permv<E>(pp[2 * kb], pp[2 * kb + 1]);
#pragma unroll
    for (int n = 0; n < 8; ++n) {
      dvl[n] = zero4();
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
        if (kb >= kb0) dvl[n] = mfma(a[kb], ld8_trp(dOs, LDK, 32 * kb, 16 * n), dvl[n]);
    }
  }
  // X^T (k-tiles 2w, 2w+1 x 8 value tiles) = (gam Q)^T dO, both read transposed
  f32x4 xt[2][8];
#pragma unroll
  for (int mm = 0; mm < 2; ++mm) {
    const int m = 2 * wave + mm;
    X8 a[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) a[kb] = to8<E>(cvtf8(ld8_tr(Qs, LDK, 32 * kb, 16 * m)) * fg[kb]);
#pragma unroll
    for (int n = 0; n < 8; ++n) {
      xt[mm][n] = zero4();
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) xt[mm][n] = mfma(a[kb], ld8_tr(dOs, LDK, 32 * kb, 16 * n), xt[mm][n]);
    }
  }
  __syncthreads();  // the input tiles are read: they take the output tiles
  E* xts = QK;      // X^T [v][k], row stride LDK
  E* dvs = dOs;     // dv_local^T [v][s], 64-element rows, 16-byte column c at c ^ (v & 7)
#pragma unroll
  for (int n = 0; n < 8; ++n) {
    const int v = 16 * n + r, sc = 2 * wave + (q4 >> 1);
    st4(dvs + v * 64 + 8 * (sc ^ (v & 7)) + 4 * (q4 & 1), dvl[n] * scale);
#pragma unroll
    for (int mm = 0; mm < 2; ++mm) st4(xts + v * LDK + 16 * (2 * wave + mm) + 4 * q4, xt[mm][n] * scale);
  }
  __syncthreads();
  {
    E* out = dvlT + cb * (D * CH);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int seg = 256 * i + tid, v = seg >> 3, part = seg & 7;
      st8(out + v * CH + 8 * part, ld8(dvs + v * 64 + 8 * (part ^ (v & 7))));
    }
  }
  {
    E* out = XT + cb * (D * D);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int seg = 256 * i + tid, v = seg >> 4, part = seg & 15;
      st8(out + v * D + 8 * part, ld8(xts + v * LDK + 8 * part));
    }
  }
  if (F16 && blockIdx.x == 0 && blockIdx.y == 0 && tid == 0) dscale[0] = ds;  // for bwd_dkw
}

// ---------------------------------------------------------------------------
// bwd_state: one wave per (head, 16-wide value slice, document), chunks in reverse
// ---------------------------------------------------------------------------
// Reverse scan, organised like fwd_scan_kernel: one consumer wave per (head,
// 16-wide value slice), two loader waves copying each chunk's operands
// global -> LDS asynchronously into a 4-stage ring, BS_DEPTH chunks ahead, each
// loader issuing its own part of every chunk (part 0: kdec Kn, G_last, X^T;
// part 1: -W^T, dv_local^T).  The consumer's output tiles (dS^T, dVn^T) go into the
// stage region it has read (-W^T) and are stored by loader 1, which refills
// that region right after.  Tiles use the same XOR swizzles as the forward
// scan:
//   Kn  [64 rows t][16 cols]   col ^ (t & 15)      W^T [128 rows k][8 cols]  col ^ ((k >> 1) & 7)
//   X^T [16 rows v][16 cols]   col ^ (v & 15)      dv_local^T [16 rows v][8 cols]  col ^ ((v >> 1) & 7)
constexpr int BS_THREADS = 64 * 3;
constexpr int BS_DEPTH = 3;
constexpr int BS_STAGES = 4;
constexpr int BS_SROW = 136;
constexpr int BS_VROW = 72;

template <class E>
struct __attribute__((aligned(16))) BwdStage {
  E kn[64 * 128];   // Kn rows t
  E wt[128 * 64];   // -W^T rows k
  E dvl[16 * 64];   // dv_local^T rows of the slice
  E xt[16 * 128];   // X^T rows of the slice
  float glast;      // G of the chunk's last event
  float pad[3];
};

template <class E>
struct __attribute__((aligned(16))) BwdScratch {
  E s[16 * BS_SROW];  // dS_{c+1}, [v][k]
  E v[16 * BS_VROW];  // dVn, [v][t]
};
static_assert(sizeof(BwdScratch<bf16>) <= 128 * 64 * sizeof(bf16), "scratch must fit the -W^T region");
template <class E>
__device__ __forceinline__ BwdScratch<E>& bwd_scratch(BwdStage<E>& st) {
  return *reinterpret_cast<BwdScratch<E>*>(st.wt);
}

// Issue part `part` of the asynchronous copies of chunk c into stage S (no
// wait on memory here): part 0 kdec Kn, G_last and the X^T slice (21 copies),
// part 1 (loader 1, which also stores the outputs) -W^T and the dv_local^T
// slice (18 copies).
constexpr int BWD_PART_COPIES[2] = {21, 18};
template <class E>
__device__ __forceinline__ void bwd_issue(BwdStage<E>& S, const int32_t* __restrict__ chunks, int c, int H, int h,
                                          int v0, int lane, int part, const E* __restrict__ knP,
                                          const float* __restrict__ gc, const E* __restrict__ dvlT,
                                          const E* __restrict__ XT, const E* __restrict__ WT) {
  const ChunkInfo ci = chunk_info(chunks, c);
  const size_t cb = (size_t)c * H + h;
  if (part == 0) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {  // rows past the tail re-read row len-1 and are zeroed by bwd_fix_tail
      const int t = 4 * i + (lane >> 4), col = (lane & 15) ^ (t & 15);
      const int tt = min(t, ci.len - 1);
      dma16(knP + ((size_t)(ci.start + tt) * H + h) * D + 8 * col, S.kn + 512 * i);
    }
    if (lane == 0)  // one lane: a dword copy writes 4 bytes per active lane
      __builtin_amdgcn_global_load_lds(gc + (size_t)(ci.start + ci.len - 1) * H + h, (lds_void_ptr)&S.glast, 4, 0,
                                       0);
    const E* xt = XT + cb * (D * D) + v0 * D;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int v = 4 * i + (lane >> 4), col = (lane & 15) ^ (v & 15);
      dma16(xt + v * D + 8 * col, S.xt + 512 * i);
    }
  } else {
    const E* wt = WT + cb * (D * CH);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int k = 8 * i + (lane >> 3), col = (lane & 7) ^ ((k >> 1) & 7);
      dma16(wt + k * CH + 8 * col, S.wt + 512 * i);
    }
    const E* dvl = dvlT + cb * (D * CH) + v0 * CH;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int v = 8 * i + (lane >> 3), col = (lane & 7) ^ ((v >> 1) & 7);
      dma16(dvl + v * CH + 8 * col, S.dvl + 512 * i);
    }
  }
}

template <class E>
__device__ __forceinline__ void bwd_fix_tail(BwdStage<E>& S, const int32_t* __restrict__ chunks, int c, int lane) {
  const int len = chunk_info(chunks, c).len;
  if (len < CH) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int t = 4 * i + (lane >> 4);
      if (t >= len) st8(S.kn + t * 128 + 8 * (lane & 15), zero8v<E>());
    }
  }
}

// global stores of one copy-out (4 of dS, 2 of dVn)
constexpr int BWD_OUT_STORES = 6;

// scratch of one step -> dS_{c+1} and dVn in value-slice-major blocks (the
// slice's [k][16] and [t][16], read transposed from the [v][k] / [v][t] scratch).
// Each store instruction writes 1 KB of contiguous lines, with the non-temporal
// hint: the scan still has the earlier chunks' operands to read (bwd_local wrote
// them first to last, so they are the oldest in the memory-side cache).  With
// bwd_dkw beside the scan (SC1) the stores are device-scope: bwd_dkw reads them
// while the scan runs.
template <bool SC1, class E>
__device__ __forceinline__ void bwd_copy_out(const BwdScratch<E>& sc, int c, int H, int h, int slice, int lane,
                                             E* __restrict__ dhS, E* __restrict__ dVnS) {
  const size_t cb = (size_t)c * H + h;
  const int r = lane & 15, q4 = lane >> 4, half = 8 * (q4 & 1), row = 16 * (q4 >> 1) + r;
  E* ds = dhS + cb * (D * D) + slice * (D * 16);
  E* vs = dVnS + cb * (CH * D) + slice * (CH * 16);
  if constexpr (SC1) {
    const __amdgpu_buffer_rsrc_t dr = buf_rsrc(ds, D * 16 * 2), vr = buf_rsrc(vs, CH * 16 * 2);
#pragma unroll
    for (int i = 0; i < 4; ++i) buf_st16_nt_sc1(dr, ((32 * i + row) * 16 + half) * 2, ld8_tr16(sc.s, BS_SROW, 32 * i));
#pragma unroll
    for (int i = 0; i < 2; ++i) buf_st16_nt_sc1(vr, ((32 * i + row) * 16 + half) * 2, ld8_tr16(sc.v, BS_VROW, 32 * i));
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) st8_nt(ds + (32 * i + row) * 16 + half, ld8_tr16(sc.s, BS_SROW, 32 * i));
#pragma unroll
    for (int i = 0; i < 2; ++i) st8_nt(vs + (32 * i + row) * 16 + half, ld8_tr16(sc.v, BS_VROW, 32 * i));
  }
}

// One slice's dS / dVn of chunk c are stored (their stores have completed): add to
// the chunk's count, which bwd_dkw waits to see at 8, from one lane.
__device__ __forceinline__ void bwd_publish(int* __restrict__ ready, int c, int H, int h, int lane) {
  asm volatile("" ::: "memory");
  if (lane == 0) count_add(ready + (size_t)c * H + h);
  asm volatile("" ::: "memory");
}

template <class E>
__global__ __launch_bounds__(BS_THREADS) void bwd_scan_kernel(
    const E* __restrict__ knP, const float* __restrict__ gc, const E* __restrict__ dvlT,
    const E* __restrict__ XT, const E* __restrict__ WT, const int32_t* __restrict__ chunks,
    const int32_t* __restrict__ doc_chunk, int H, E* __restrict__ dhS, E* __restrict__ dVnS,
    int* __restrict__ ready, int* __restrict__ resident) {
  // ready / resident: null, or the hand-off counts of a bwd_dkw running beside this
  // scan (each workgroup adds one to resident when it starts, and one to a chunk's
  // ready count once its outputs of that chunk are stored)
  typedef typename Vec<E>::x8 X8;
  typedef typename Vec<E>::x4 X4;
  const int h = blockIdx.x % H, slice = blockIdx.x / H, d = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q4 = lane >> 4;
  const int v0 = 16 * slice;

  __shared__ BwdStage<E> stage[BS_STAGES];

  const int c_end = doc_chunk[d + 1], n = c_end - doc_chunk[d];
  // step tau handles chunk c_end - 1 - tau (chunks in reverse)
  if (wave == 0) {
    if (resident && lane == 0) count_add(resident);
    f32x4 dS[8];  // dS[m][i] = dState[k = 16m + 4q4 + i][v = v0 + r]
#pragma unroll
    for (int m = 0; m < 8; ++m) dS[m] = zero4();
    int kofs[4], wofs[2], dofs[4], xofs[8];
#pragma unroll
    for (int j = 0; j < 4; ++j) kofs[j] = 2 * (r * 128 + 8 * ((4 * j + q4) ^ r));
#pragma unroll
    for (int j = 0; j < 2; ++j) wofs[j] = 2 * (r * 64 + 8 * ((4 * j + q4) ^ ((r >> 1) & 7)));
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) dofs[i4] = 2 * (r * 64 + 8 * ((2 * i4 + (q4 >> 1)) ^ ((r >> 1) & 7)) + 4 * (q4 & 1));
#pragma unroll
    for (int m = 0; m < 8; ++m) xofs[m] = 2 * (r * 128 + 8 * ((2 * m + (q4 >> 1)) ^ r) + 4 * (q4 & 1));
    const int sofs = 2 * (r * BS_SROW + 4 * q4), vofs = 2 * (r * BS_VROW + 4 * q4);
    for (int tau = -BS_DEPTH; tau < n; ++tau) {
      if (tau >= 0) {
        char* base = reinterpret_cast<char*>(&stage[tau & (BS_STAGES - 1)]);
        const char* knb = base + offsetof(BwdStage<E>, kn);
        const char* wtb = base + offsetof(BwdStage<E>, wt);
        const char* dvb = base + offsetof(BwdStage<E>, dvl);
        const char* xtb = base + offsetof(BwdStage<E>, xt);
        // every operand read is issued ahead of the MFMAs that use them (the
        // kdec Kn fragments first); the scheduling barriers keep the compiler
        // from interleaving them one by one
        X8 fk[4][4], fw[8][2];
        f32x4 xv[8];
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int i4 = 0; i4 < 4; ++i4) fk[i4][j] = *reinterpret_cast<const X8*>(knb + kofs[j] + 4096 * i4);
        // dVn = dv_local + (kdec Kn) dS_{c+1}, accumulated onto dv_local
        f32x4 dv[4];
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) dv[i4] = cvtf4(*reinterpret_cast<const X4*>(dvb + dofs[i4]));
        const float glast = reinterpret_cast<const BwdStage<E>*>(base)->glast;
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int m = 0; m < 8; ++m) fw[m][j] = *reinterpret_cast<const X8*>(wtb + wofs[j] + 2048 * m);
#pragma unroll
        for (int m = 0; m < 8; ++m) xv[m] = cvtf4(*reinterpret_cast<const X4*>(xtb + xofs[m]));
        __builtin_amdgcn_sched_barrier(0);
        X4 sh[8];
#pragma unroll
        for (int m = 0; m < 8; ++m) sh[m] = to4<E>(dS[m]);
        // beside it, the first two terms of dS_c = exp(G_last) dS_{c+1} + X + (-W^T) dVn
        const float gC = __expf(glast);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const X8 sb = cat(sh[2 * j], sh[2 * j + 1]);
#pragma unroll
          for (int i4 = 0; i4 < 4; ++i4) dv[i4] = mfma(fk[i4][j], sb, dv[i4]);
#pragma unroll
          for (int m = 2 * j; m < 2 * j + 2; ++m) dS[m] = dS[m] * gC + xv[m];
        }
        __builtin_amdgcn_sched_barrier(0);
        // the -W^T fragments have been read (a wave's LDS operations complete in
        // order): the -W^T region now takes this step's outputs
        char* sb = base + offsetof(BwdStage<E>, wt);
#pragma unroll
        for (int m = 0; m < 8; ++m) *reinterpret_cast<X4*>(sb + sofs + 32 * m) = sh[m];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const X8 nb = pack_permv<E>(dv[2 * j], dv[2 * j + 1]);
#pragma unroll
          for (int m = 0; m < 8; ++m) dS[m] = mfma(fw[m][j], nb, dS[m]);
        }
        char* vbp = sb + sizeof(BwdScratch<E>::s);
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) *reinterpret_cast<X4*>(vbp + vofs + 32 * i4) = to4<E>(dv[i4]);
      }
      lds_barrier();
    }
  } else {
    // Step tau, both loaders: wait for their part of step tau+1's chunk, then
    // refill stage (tau-1)%4 with their part of step tau+3's chunk (loader 1
    // first stores step tau-1's outputs from that stage's -W^T region).  Loads
    // and stores retire in issue order, so a loader waits by letting exactly
    // the operations it issued after that part stay in flight (as in the
    // forward scan).  Loader 1's wait at step tau >= 3 also covers the copy-out
    // of step tau-3 (issued before step tau+1's part), so with a bwd_dkw beside
    // the scan it then announces that step's chunk: one atomic add, in flight
    // with the step's other operations and counted in the next wait.
    const int j = wave - 1;
    for (int tau = -BS_DEPTH; tau < n; ++tau) {
      const int xn = tau + 1, xo = tau - 1, xi = tau + BS_DEPTH;
      if (xn >= 0 && xn < n) {
        const bool later = xn + 1 < n;  // this loader's part of step tau+2's chunk is in flight
        if (j == 0) {
          if (later)
            wait_vmem_le<BWD_PART_COPIES[0]>();
          else
            wait_vmem_all();
          bwd_fix_tail(stage[xn & (BS_STAGES - 1)], chunks, c_end - 1 - xn, lane);
        } else {
          const bool stored = tau >= 2;                 // the copy-out of step tau-2 came after this part
          const bool announced = ready && tau >= 4;     // and step tau-1's announcement (of step tau-4)
          if (later && announced)
            wait_vmem_le<BWD_PART_COPIES[1] + BWD_OUT_STORES + 1>();
          else if (later && stored)
            wait_vmem_le<BWD_PART_COPIES[1] + BWD_OUT_STORES>();
          else if (later)
            wait_vmem_le<BWD_PART_COPIES[1]>();
          else if (announced)
            wait_vmem_le<BWD_OUT_STORES + 1>();
          else if (stored)
            wait_vmem_le<BWD_OUT_STORES>();
          else
            wait_vmem_all();
          if (ready && tau >= 3) bwd_publish(ready, c_end - 1 - (tau - 3), H, h, lane);
        }
      }
      if (j == 1 && xo >= 0) {
        if (ready)
          bwd_copy_out<true>(bwd_scratch(stage[xo & (BS_STAGES - 1)]), c_end - 1 - xo, H, h, slice, lane, dhS, dVnS);
        else
          bwd_copy_out<false>(bwd_scratch(stage[xo & (BS_STAGES - 1)]), c_end - 1 - xo, H, h, slice, lane, dhS, dVnS);
      }
      if (xi < n)
        bwd_issue(stage[xi & (BS_STAGES - 1)], chunks, c_end - 1 - xi, H, h, v0, lane, j, knP, gc, dvlT, XT, WT);
      lds_barrier();
    }
    if (n > 0 && j == 1) {
      if (ready)
        bwd_copy_out<true>(bwd_scratch(stage[(n - 1) & (BS_STAGES - 1)]), c_end - n, H, h, slice, lane, dhS, dVnS);
      else
        bwd_copy_out<false>(bwd_scratch(stage[(n - 1) & (BS_STAGES - 1)]), c_end - n, H, h, slice, lane, dhS, dVnS);
      if (ready) {
        // the loop announced steps 0 .. n-5; the rest once every store has completed
        wait_vmem_all();
        for (int s = max(n - 4, 0); s < n; ++s) bwd_publish(ready, c_end - 1 - s, H, h, lane);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// bwd_dkw: the dq/dK/dW part and then the WY part in one workgroup per (chunk, head), so the
// dK partial (registers), dW (LDS), the dG partial (a register of wave 0) and the
// K tile never leave the chip.  LDS regions are reused as their first users die
// (81,408 bytes: two workgroups per CU):
//   R1  Q rows            -> V rows (wy)
//   R2  K rows            (both parts)
//   R3  dPm^T             -> T (wy)
//   R4a dO rows           -> dVn tile (value-slice-major) + q.dq row dots
//                         -> dT^T / (beta dM)^T staging + beta, dbeta and k.dK partials (wy)
//   R4b v_new^T           -> dW rows [t][k]   -> Y^T staging (wy)
// dPm and the wy staging tiles are stored transposed: an MFMA result fragment
// holds 4 consecutive rows of one column per lane, which then leave as one
// 8-byte write instead of four 2-byte writes (readers swap row and transposed
// reads accordingly).
// The l2norm backward of dq runs on the phase-2 registers (per-wave row dots in
// LDS), so no fp32 staging tile is needed and dQ's registers carry the dK partial.
// Barriers order LDS only (s_waitcnt lgkmcnt(0); s_barrier): global stores stay
// in flight across them, and the one barrier that needs the dVn tile's copies
// waits for vector memory explicitly.
constexpr int DKW_R1 = 0, DKW_R2 = 64 * LDK * 2, DKW_R3 = DKW_R2 + 64 * LDK * 2, DKW_R4A = DKW_R3 + 64 * LDT * 2,
              DKW_R4B = DKW_R4A + 64 * LDK * 2, DKW_BYTES = DKW_R4B + 128 * LDT * 2;

template <class E>  // dscale, vscale: null in bf16; in fp16 the device scalars s_d and s_v
__global__ __launch_bounds__(256, 2) void bwd_dkw_kernel(
    const E* __restrict__ q, const E* __restrict__ k,
    const float* __restrict__ rk, const float* __restrict__ gc, const E* __restrict__ hT,
    const E* __restrict__ vnT, const E* __restrict__ dout, const E* __restrict__ dh,
    const E* __restrict__ dVn, const E* __restrict__ vin, const float* __restrict__ beta,
    const E* __restrict__ Tm, const int32_t* __restrict__ chunks, int H, float scale, int normalize,
    const float* __restrict__ dscale, const float* __restrict__ vscale,
    E* __restrict__ dq, E* __restrict__ dk, E* __restrict__ dv, float* __restrict__ dg,
    float* __restrict__ dbeta, const int* __restrict__ ready, int ready_target, int ready_polls) {
  // grid (H, NC).  After the reverse scan: chunks first to last (the scan wrote the
  // first chunks last, so they are the likeliest still in the memory-side cache).
  // Beside the scan (ready != null): chunks last to first, the order the scan
  // finishes them, each workgroup waiting for its chunk's count after phase 1.
  typedef typename Vec<E>::x8 X8;
  constexpr bool F16 = __is_same(E, f16);
  // fp16: dq, dk, dg and dbeta leave divided by s_d s_v, dv by s_d (powers of two: exact)
  float inv_dv = 1.f, inv_d = 1.f, vs = 1.f;
  if constexpr (F16) {
    vs = *vscale;
    inv_d = 1.f / *dscale;
    inv_dv = inv_d / vs;
  }
  const HeadChunk hc = xcd_head_chunk(gridDim.x, gridDim.y);  // all heads of a chunk on one XCD
  const int h = hc.h, c = ready ? gridDim.y - 1 - hc.p : hc.p;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, q4 = lane >> 4;
  const ChunkInfo ci = chunk_info(chunks, c);
  const size_t cb = (size_t)c * H + h;

  // One array per region: the compiler then sees that the dVn tile's
  // asynchronous copy writes R4a only, and lets phase 3's reads of the other
  // regions run while it is in flight (with a single array it waited for the
  // copy, and every store before it, ahead of phase 3's first LDS read).
  __shared__ __attribute__((aligned(16))) uint8_t r1[DKW_R2 - DKW_R1];
  __shared__ __attribute__((aligned(16))) uint8_t r2[DKW_R3 - DKW_R2];
  __shared__ __attribute__((aligned(16))) uint8_t r3[DKW_R4A - DKW_R3];
  __shared__ __attribute__((aligned(16))) uint8_t r4a[DKW_R4B - DKW_R4A];
  __shared__ __attribute__((aligned(16))) uint8_t r4b[DKW_BYTES - DKW_R4B];
  __shared__ __attribute__((aligned(16))) float Gs[64];
  __shared__ float dgw[4][64];
  __shared__ __attribute__((aligned(16))) float Rs[64];  // rsqrt norms of q (1 without normalize)
  __shared__ int stale_s;  // nonzero when the wait for the reverse scan gave up
  E* Qs = reinterpret_cast<E*>(r1);
  E* Ks = reinterpret_cast<E*>(r2);
  E* dPm = reinterpret_cast<E*>(r3);
  E* dOs = reinterpret_cast<E*>(r4a);
  E* VnT = reinterpret_cast<E*>(r4b);  // v_new^T [v][t], read transposed as v_new rows
  E* dVs = dOs;                        // dVn tile, from phase 3 on
  float* dqdot = reinterpret_cast<float*>(r4a + CH * D * 2);  // [64][4 waves] after the dVn tile
  E* dWs = VnT;                        // dW rows [t][k], from phase 4 on

  // This wave's state fragments: rows k = 16 (2 wave + mm) + r of h
  // (column gathers of h^T) and of dS_{c+1}, value block kb.
  const E* ht = hT + cb * (D * D);
  X8 bh[2][4], bd[2][4];
  // Every prologue load is issued before the first wait: the column gathers'
  // loads, the gate and k-norm values (unconditional: rk is allocated either
  // way), the v_new^T rows and the Q, K, dO rows; the gathers' lane exchange
  // comes last.  The q norm is formed from the Q rows (row_rnorm).
  {
    Col8 gh[2][4];
#pragma unroll
    for (int mm = 0; mm < 2; ++mm)
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) gh[mm][kb] = col8_load(ht, D, 32 * kb, 16 * (2 * wave + mm));
    const int t = tid >> 2, p = tid & 3;
    const bool in = t < ci.len;
    const int tc = clamp_row(t, ci.len);
    const size_t ev = (size_t)(ci.start + tc) * H + h, row = ev * D;
    const float gv = gc[ev];
    const float rkv = rk[ev];
    const E* vt = vnT + cb * (D * CH);
    X8 xv[4], xq[4], xk[4], xo[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int seg = 256 * i + tid, v = seg >> 3, part = seg & 7;
      xv[i] = ld8(vt + v * CH + 8 * part);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int col = 32 * j + 8 * p;
      xq[j] = ld8(q + row + col);
      xk[j] = ld8(k + row + col);
      xo[j] = ld8(dout + row + col);
    }
    dgw[wave][lane] = 0.f;
    const float rv = normalize ? row_rnorm(xq) : 1.f;
    if (p == 0) {
      Gs[t] = gv;
      Rs[t] = rv;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int seg = 256 * i + tid, v = seg >> 3, part = seg & 7;
      st8(VnT + v * LDT + 8 * part, xv[i]);
    }
    if constexpr (F16) {  // dO s_d (exact: a power of two, in range)
      const float ds = *dscale;
#pragma unroll
      for (int j = 0; j < 4; ++j) xo[j] = to8<E>(cvtf8(xo[j]) * ds);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int col = 32 * j + 8 * p;
      st8(Qs + t * LDK + col, keep_if(in, scaled8<E>(xq[j], rv)));
      st8(Ks + t * LDK + col, keep_if(in, scaled8<E>(xk[j], rkv)));
      st8(dOs + t * LDK + col, keep_if(in, xo[j]));
    }
#pragma unroll
    for (int mm = 0; mm < 2; ++mm)
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) bh[mm][kb] = col8_combine_v<E>(gh[mm][kb]);
  }
  lds_barrier();
  const float glast = Gs[ci.len - 1];
  float* dgl = dgw[wave];

  // ---- phase 1: P, dP over the ten causal (t-tile, s-tile) pairs: wave w takes t-tile w with
  //      s-tiles 0 .. min(w, 2) and wave 0 also the (3, 3) diagonal, at most three pairs a wave ----
  // The gates Gam[t][s] of this wave's pairs stay in registers for the wy phase 3, which
  // takes the same pairs in the same fragment layout: gk[n] for s-tile n of t-tile wave,
  // gk[3] for wave 0's (3, 3) tile.
  f32x4 gk[4];
  {
    // dPm of t-tile tt, s-tile n; its row sums are added to rowE, its column sums to dgl
    auto pair = [&](int tt, int n, float(&rowE)[4], f32x4& gout) -> f32x4 {
      f32x4 p = zero4(), dp = zero4();
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        p = mfma(ld8(Qs + (16 * tt + r) * LDK + 32 * kb + 8 * q4), ld8(Ks + (16 * n + r) * LDK + 32 * kb + 8 * q4), p);
        dp = mfma(ld8(dOs + (16 * tt + r) * LDK + 32 * kb + 8 * q4), ld8_tr(VnT, LDT, 32 * kb, 16 * n), dp);
      }
      const int s = 16 * n + r;
      const f32x4 g4 = *reinterpret_cast<const f32x4*>(&Gs[16 * tt + 4 * q4]);
      const float gs = Gs[s];
      float colE = 0.f;
      f32x4 dpm;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = 16 * tt + 4 * q4 + i;
        const float gam = (s <= t) ? __expf(g4[i] - gs) : 0.f;
        gout[i] = gam;
        dpm[i] = scale * dp[i] * gam;
        const float e = dpm[i] * p[i];
        rowE[i] += e;
        colE += e;
      }
      colE = sum_rows4(colE);
      if (q4 == 0) dgl[s] -= colE;
      return dpm;
    };
    float rowE[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      if (n == 3 && wave == 3) continue;  // the (3, 3) tile is wave 0's
      const f32x4 dpm = (n <= wave) ? pair(wave, n, rowE, gk[n]) : zero4();
      st4(dPm + (16 * n + r) * LDT + 16 * wave + 4 * q4, dpm);  // transposed: dPm^T[s][t], 4 rows t in 8 bytes
    }
    sum16x4(rowE);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (r == 0) dgl[16 * wave + 4 * q4 + i] += rowE[i];
    if (wave == 0) {
      float rowE3[4] = {0.f, 0.f, 0.f, 0.f};
      st4(dPm + (48 + r) * LDT + 48 + 4 * q4, pair(3, 3, rowE3, gk[3]));
      sum16x4(rowE3);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (r == 0) dgl[48 + 4 * q4 + i] += rowE3[i];
    }
  }
  // dS_{c+1} and dVn are the reverse scan's: beside it, wait until all eight value
  // slices of this chunk are stored (wave 1 has the fewest phase-1 pairs).  If the
  // wait gives up, dS_{c+1} and dVn are taken as NaN, which turns every output that
  // depends on them (dk, dv, dg, dbeta) to NaN; dq does not depend on them.
  if (wave == 1) {
    bool ok = true;
    if (ready && lane == 0) ok = count_wait_ge(ready + cb, ready_target, ready_polls);
    if (lane == 0) stale_s = ok ? 0 : 1;
  }
  lds_barrier();
  const bool stale = stale_s != 0;
  const __amdgpu_buffer_rsrc_t dh_rs = buf_rsrc(dh + cb * (D * D), D * D * 2);

  // (device-scope loads beside the scan, which may still be running)
#pragma unroll
  for (int mm = 0; mm < 2; ++mm)
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const int i = (2 * kb + (q4 >> 1)) * (D * 16) + (16 * (2 * wave + mm) + r) * 16 + 8 * (q4 & 1);
      bd[mm][kb] = ready ? buf_ld16_sc1<X8>(dh_rs, i * 2) : ld8(dh + cb * (D * D) + i);
    }
  if (stale) {
    asm volatile("");  // a branch, not selects
#pragma unroll
    for (int mm = 0; mm < 2; ++mm)
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) bd[mm][kb] = to8<E>(f32x8{NAN, NAN, NAN, NAN, NAN, NAN, NAN, NAN});
  }

  // ---- phase 2: dQ^T (k-tiles 2w, 2w+1 as rows, t columns); dG_t from the output term ----
  // Each MFMA takes the operands of dQ = dO h^T + (dP Gam) K swapped, so a lane holds 4
  // consecutive k of one row t: dQ[mm][n][i] = dq[t = 16 n + r][k = 16 (2w + mm) + 4 q4 + i].
  // The row's gate and norm are then one value per lane, its sums over k run over the
  // 4 lanes of a column (permlane swaps), and dq leaves as 8-byte pieces of rows.
  f32x4 dQ[2][4];
  f32x4 qrow[4][2];  // q[t = 16 n + r][k = 16 (2w + mm) + 4 q4 + i], kept for the dq stores
  float pdot[4];     // this wave's parts of the row dots q_t . dQ_t (l2norm backward of dq)
  {
    f32x4 a1[2][4];
#pragma unroll
    for (int mm = 0; mm < 2; ++mm)
#pragma unroll
      for (int n = 0; n < 4; ++n) a1[mm][n] = dQ[mm][n] = zero4();
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        const X8 a = ld8(dOs + (16 * n + r) * LDK + 32 * kb + 8 * q4);
#pragma unroll
        for (int mm = 0; mm < 2; ++mm) a1[mm][n] = mfma(bh[mm][kb], a, a1[mm][n]);
      }
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        if (n < 2 * kb) continue;
        const X8 a = ld8_tr(dPm, LDT, 32 * kb, 16 * n);  // dPm rows t = 16 n + r
#pragma unroll
        for (int mm = 0; mm < 2; ++mm)
          dQ[mm][n] = mfma(ld8_tr(Ks, LDK, 32 * kb, 16 * (2 * wave + mm)), a, dQ[mm][n]);
      }
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      const float f = scale * __expf(Gs[16 * n + r]);
#pragma unroll
      for (int mm = 0; mm < 2; ++mm) qrow[n][mm] = cvtf4(ld4(Qs + (16 * n + r) * LDK + 16 * (2 * wave + mm) + 4 * q4));
      float x = 0.f, y = 0.f;  // x: the output term's dG_t part; y: q_t . dQ_t (dQ complete here)
#pragma unroll
      for (int mm = 0; mm < 2; ++mm)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float inter = a1[mm][n][i] * f;
          dQ[mm][n][i] += inter;
          x += qrow[n][mm][i] * inter;
          y += qrow[n][mm][i] * dQ[mm][n][i];
        }
      x = sum_rows4(x);
      if (q4 == 0) dgl[16 * n + r] += x;
      pdot[n] = sum_rows4(y);
    }
  }
  lds_barrier();  // every read of the dO rows is done: the row dots and then the dVn tile may replace them
  if (q4 == 0) {
#pragma unroll
    for (int n = 0; n < 4; ++n) dqdot[4 * (16 * n + r) + wave] = pdot[n];  // after the tile's 16 KB
  }
  lds_barrier();
  // The dS fragments (bd) requested after phase 1 have landed long since: wait
  // for them here, where nothing else is in flight, so that their first use in
  // phase 3 does not wait for the dq stores and the dVn copy issued below (the
  // stores are conditional, so the compiler could only wait for everything).
  wait_vmem_all();
  // dq = rq (dQ - q (q . dQ)): each lane stores 4 consecutive k of row t = 16 n + r
  const int rowb = H * D * 2;  // bytes per event row
  {
  const __amdgpu_buffer_rsrc_t dq_rs = chunk_rows_rsrc(dq, ci.start, ci.len, H, h);
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    const int t = 16 * n + r;
    const float rs = Rs[t];
    const f32x4 d4 = *reinterpret_cast<const f32x4*>(&dqdot[4 * t]);
    const float dot = d4[0] + d4[1] + d4[2] + d4[3];
#pragma unroll
    for (int mm = 0; mm < 2; ++mm) {
      const int k0 = 16 * (2 * wave + mm) + 4 * q4;
      const f32x4 x = normalize ? (dQ[mm][n] - qrow[n][mm] * dot) * rs : dQ[mm][n];
      buf_st4<E>(dq_rs, r * rowb + k0 * 2, 16 * n * rowb, F16 ? x * inv_dv : x);  // row t, columns k0 .. k0 + 3
    }
  }
  }
  // the dVn tile, copied global -> LDS while phase 3 runs (after the dq stores, which retire first)
  {
    const E* dvs = dVn + cb * (CH * D);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (stale)
        st8(dVs + 512 * (4 * i + wave) + 8 * lane, to8<E>(f32x8{NAN, NAN, NAN, NAN, NAN, NAN, NAN, NAN}));
      else if (ready)
        dma16_sc1(dvs + 512 * (4 * i + wave) + 8 * lane, dVs + 512 * (4 * i + wave));
      else
        dma16(dvs + 512 * (4 * i + wave) + 8 * lane, dVs + 512 * (4 * i + wave));
    }
  }

  // ---- phase 3: dK^T partial (k rows, t columns), kept in registers for the wy part ----
  f32x4 fkp[2][4];
  {
    float esum = 0.f;
#pragma unroll
    for (int mm = 0; mm < 2; ++mm) {
      const int m = 2 * wave + mm;
      f32x4 a3[4], a4[4];
#pragma unroll
      for (int n = 0; n < 4; ++n) a3[n] = a4[n] = zero4();
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const X8 a = ld8_tr(Qs, LDK, 32 * kb, 16 * m);
#pragma unroll
        for (int n = 0; n < 4; ++n) {
          if (n > 2 * kb + 1) continue;
          a3[n] = mfma(a, ld8(dPm + (16 * n + r) * LDT + 32 * kb + 8 * q4), a3[n]);  // dPm^T rows s
        }
      }
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
#pragma unroll
        for (int n = 0; n < 4; ++n) a4[n] = mfma(bd[mm][kb], ld8_tr(VnT, LDT, 32 * kb, 16 * n), a4[n]);
      }
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        const int t = 16 * n + r;
        const float kd = __expf(glast - Gs[t]);
        const f32x4 st = a4[n] * kd;
        const f32x4 kk = cvtf4(ld4(Ks + t * LDK + 16 * m + 4 * q4));
        float e = st[0] * kk[0] + st[1] * kk[1] + st[2] * kk[2] + st[3] * kk[3];
        e = sum_rows4(e);
        if (q4 == 0) dgl[t] -= e;
        esum += (q4 == 0) ? e : 0.f;
        fkp[mm][n] = keep_if(t < ci.len, a3[n] + st);
      }
    }
    esum = sum16(esum);
    // <h, dS_{c+1}> over this wave's quarter of both
    float x = 0.f;
#pragma unroll
    for (int mm = 0; mm < 2; ++mm)
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) x = dot8(bh[mm][kb], bd[mm][kb], x);
    x = sum16(x);
    x = sum_rows4(x);
    if (lane == 0) dgl[ci.len - 1] += esum + __expf(glast) * x;
  }
  wait_vmem_all();  // the dVn tile has landed (the dq stores issued before it have retired too)
  lds_barrier();    // every read of Q, dPm and v_new^T is done

  // the wy part's V rows, T rows and beta, requested now and stored over Q and dPm after phase 4
  X8 pv[4], pt[2];
  float pb;
  {
    const int t = tid >> 2, p = tid & 3;
    const bool in = t < ci.len;
    const int tc = clamp_row(t, ci.len);
    const size_t row = ((size_t)(ci.start + tc) * H + h) * D;
    pb = keep_if(in, beta[(size_t)(ci.start + tc) * H + h]);
#pragma unroll
    for (int j = 0; j < 4; ++j) pv[j] = keep_if(in, ld8(vin + row + 32 * j + 8 * p));
    const E* tm = Tm + cb * (CH * CH);
#pragma unroll
    for (int j = 0; j < 2; ++j) pt[j] = ld8(tm + t * CH + 32 * j + 8 * p);
  }

  // ---- phase 4: dW = -dVn S^T into LDS rows [t][k]; the wy part's dVn fragments ----
  X8 fdv[4], fvt[2][2];
  {
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      const int t = 16 * n + r;
      X8 av[4];  // dVn row t, value block kb
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) av[kb] = ld8(dVs + (2 * kb + (q4 >> 1)) * (CH * 16) + t * 16 + 8 * (q4 & 1));
#pragma unroll
      for (int mm = 0; mm < 2; ++mm) {
        const int m = 2 * wave + mm;
        f32x4 w = zero4();  // -dW^T[k = 16 m + 4 q4 + i][t] = (dVn S^T)^T, zero past the chunk
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) w = mfma(bh[mm][kb], av[kb], w);
        st4(dWs + t * LDK + 16 * m + 4 * q4, keep_if(t < ci.len, w));
      }
    }
    const int t = 16 * wave + r;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
      fdv[kb] = keep_if(t < ci.len, ld8(dVs + (2 * kb + (q4 >> 1)) * (CH * 16) + t * 16 + 8 * (q4 & 1)));
#pragma unroll
    for (int mm = 0; mm < 2; ++mm)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) fvt[mm][kb] = ld8_tr(dVs + (2 * wave + mm) * (CH * 16), 16, 32 * kb, 0);
  }
  lds_barrier();  // -dW rows complete, dG partials complete, the dVn tile consumed

  // ---- the WY part, on the chip-resident operands ----
  const float dgp_t = (tid < 64) ? dgw[0][tid] + dgw[1][tid] + dgw[2][tid] + dgw[3][tid] : 0.f;
  E* Vs = Qs;
  E* Ts = dPm;
  E* S1 = dOs;  // transposed: dT^T[s][t], then (beta dM)^T [j][i]
  E* S2 = VnT;                                                              // Y^T[j][t], over dW rows
  float* Bs = reinterpret_cast<float*>(r4a + 64 * LDT * 2);                   // after S1
  float* dbw = Bs + 64;                                                        // [4][64]
  float* dkdot = dbw + 256;                                                    // [64][4 waves]
  {
    const int t = tid >> 2, p = tid & 3;
    if (p == 0) Bs[t] = pb;
#pragma unroll
    for (int j = 0; j < 4; ++j)  // fp16: V s_v, in the scale of the forward's v_new and U
      st8(Vs + t * LDK + 32 * j + 8 * p, F16 ? to8<E>(cvtf8(pv[j]) * vs) : pv[j]);
#pragma unroll
    for (int j = 0; j < 2; ++j) st8(Ts + t * LDT + 32 * j + 8 * p, pt[j]);
  }
  lds_barrier();  // dgp_t has been read everywhere it is needed
  dgw[wave][lane] = 0.f;
  dbw[wave * 64 + lane] = 0.f;
  lds_barrier();
  float* dbl = dbw + wave * 64;

  // ---- wy phase 1: dT = dW (beta gam K)^T + dVn (beta V)^T -> S1 = dT[t][s]; dW fragments ----
  X8 fwt[2][2];
#pragma unroll
  for (int mm = 0; mm < 2; ++mm)
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) fwt[mm][kb] = ld8_tr(dWs, LDK, 32 * kb, 16 * (2 * wave + mm));
  {
    X8 fdw[4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) fdw[kb] = ld8(dWs + (16 * wave + r) * LDK + 32 * kb + 8 * q4);
    f32x4 ak[4], av[4];
#pragma unroll
    for (int n = 0; n < 4; ++n) ak[n] = av[n] = zero4();
#pragma unroll
    for (int kb = 0; kb < 4; ++kb)
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        ak[n] = mfma(fdw[kb], ld8(Ks + (16 * n + r) * LDK + 32 * kb + 8 * q4), ak[n]);
        av[n] = mfma(fdv[kb], ld8(Vs + (16 * n + r) * LDK + 32 * kb + 8 * q4), av[n]);
      }
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      const int s = 16 * n + r;
      const float fk = -(Bs[s] * __expf(Gs[s])), fv = Bs[s];  // ak holds -dW (beta gam K)^T
      st4(S1 + s * LDT + 16 * wave + 4 * q4, ak[n] * fk + av[n] * fv);
    }
  }
  float rsn[4];
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    const float x = rk[(size_t)(ci.start + clamp_row(16 * n + r, ci.len)) * H + h];  // allocated either way
    rsn[n] = normalize ? x : 1.f;
  }
  lds_barrier();  // S1 complete; every wave holds its dW fragments (S2 may overwrite the rows)

  // ---- wy phase 2: Y = dT T^T -> S2 = Y^T[j][t] ----
  {
    X8 a[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) a[kb] = ld8_tr(S1, LDT, 32 * kb, 16 * wave);  // dT rows t = 16 wave + r
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      f32x4 acc = zero4();
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        if (n < 2 * kb) continue;  // T[j][b] = 0 for b > j
        acc = mfma(a[kb], ld8(Ts + (16 * n + r) * LDT + 32 * kb + 8 * q4), acc);
      }
      st4(S2 + (16 * n + r) * LDT + 16 * wave + 4 * q4, acc);
    }
  }
  lds_barrier();

  // ---- wy phase 3: dA = -T^T Y, dM, dbeta and dG from A, over the causal (i-tile, j-tile) pairs
  //      shared out as in phase 1 ----
  {
    // (beta dM)^T of i-tile it, j-tile n (at, ak: T^T and K fragments of i-tile it; gam: the
    // tile's gates from phase 1, whose diagonal 1 is masked here by dA's strict mask)
    auto pair = [&](int it, int n, const X8(&at)[2], const X8(&ak)[4], const f32x4& gam,
                    float(&rowB)[4], float(&rowE)[4]) -> f32x4 {
      f32x4 da = zero4(), kk = zero4();
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
        if (kb >= (it >= 2 ? 1 : 0)) da = mfma(at[kb], ld8(S2 + (16 * n + r) * LDT + 32 * kb + 8 * q4), da);
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) kk = mfma(ak[kb], ld8(Ks + (16 * n + r) * LDK + 32 * kb + 8 * q4), kk);
      const int j = 16 * n + r;
      const f32x4 b4 = *reinterpret_cast<const f32x4*>(&Bs[16 * it + 4 * q4]);
      float colE = 0.f;
      f32x4 dmp;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int i = 16 * it + 4 * q4 + e;
        const bool strict = j < i;
        const float dA = strict ? -da[e] : 0.f;
        const float dM = dA * gam[e];
        const float Aij = b4[e] * kk[e] * gam[e];
        dmp[e] = b4[e] * dM;
        rowB[e] += dM * kk[e];
        const float e2 = dA * Aij;
        rowE[e] += e2;
        colE += e2;
      }
      colE = sum_rows4(colE);
      if (q4 == 0) dgl[j] -= colE;
      return dmp;
    };
    auto rows = [&](int it, const float(&rowB)[4], const float(&rowE)[4]) {
      float xb[4] = {rowB[0], rowB[1], rowB[2], rowB[3]}, xe[4] = {rowE[0], rowE[1], rowE[2], rowE[3]};
      sum16x4(xb);
      sum16x4(xe);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (r == 0) {
          dbl[16 * it + 4 * q4 + e] += xb[e];
          dgl[16 * it + 4 * q4 + e] += xe[e];
        }
      }
    };
    {
      X8 at[2], ak[4];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) at[kb] = ld8_tr(Ts, LDT, 32 * kb, 16 * wave);
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) ak[kb] = ld8(Ks + (16 * wave + r) * LDK + 32 * kb + 8 * q4);
      float rowB[4] = {0.f, 0.f, 0.f, 0.f}, rowE[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        if (n == 3 && wave == 3) continue;  // the (3, 3) tile is wave 0's
        const f32x4 dmp = (n <= wave) ? pair(wave, n, at, ak, gk[n], rowB, rowE) : zero4();
        st4(S1 + (16 * n + r) * LDT + 16 * wave + 4 * q4, dmp);
      }
      rows(wave, rowB, rowE);
    }
    if (wave == 0) {
      X8 at[2], ak[4];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) at[kb] = ld8_tr(Ts, LDT, 32 * kb, 48);
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) ak[kb] = ld8(Ks + (48 + r) * LDK + 32 * kb + 8 * q4);
      float rowB[4] = {0.f, 0.f, 0.f, 0.f}, rowE[4] = {0.f, 0.f, 0.f, 0.f};
      st4(S1 + (48 + r) * LDT + 48 + 4 * q4, pair(3, 3, at, ak, gk[3], rowB, rowE));
      rows(3, rowB, rowE);
    }
  }
  lds_barrier();

  // The norms rsn requested in wy phase 1 have landed: wait here, before the
  // conditional dv stores, so that phase 5 does not wait for those stores.
  wait_vmem_all();
  // ---- wy phase 4b: dv = beta (T^T dVn) ----
  {
    const __amdgpu_buffer_rsrc_t dv_rs = chunk_rows_rsrc(dv, ci.start, ci.len, H, h);
    float colB[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int mm = 0; mm < 2; ++mm) {
      const int m = 2 * wave + mm;
      f32x4 acc[4];
#pragma unroll
      for (int n = 0; n < 4; ++n) acc[n] = zero4();
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const X8 a = fvt[mm][kb];
#pragma unroll
        for (int n = 0; n < 4; ++n)
          if (kb >= 1 || n < 2) acc[n] = mfma(a, ld8_tr(Ts, LDT, 32 * kb, 16 * n), acc[n]);
      }
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        const int s = 16 * n + r;
        const f32x4 vv = cvtf4(ld4(Vs + s * LDK + 16 * m + 4 * q4));
        colB[n] += acc[n][0] * vv[0] + acc[n][1] * vv[1] + acc[n][2] * vv[2] + acc[n][3] * vv[3];
        buf_st4<E>(dv_rs, r * rowb + (16 * m + 4 * q4) * 2, 16 * n * rowb,
                   acc[n] * (F16 ? Bs[s] * inv_d : Bs[s]));  // row s
      }
    }
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      float xb = colB[n];
      xb = sum_rows4(xb);
      if (q4 == 0) dbl[16 * n + r] += xb;
    }
  }

  // ---- wy phase 4a: dK in registers ----
  f32x4 dkr[2][4];
  f32x4 krow[4][2];  // k[t = 16 n + r][16 (2w + mm) + 4 q4 + i], kept for the dk stores
  float pdk[4] = {0.f, 0.f, 0.f, 0.f};  // this wave's parts of the row dots k_t . dK_t
  {
    float colB[4] = {0.f, 0.f, 0.f, 0.f}, colG[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int mm = 0; mm < 2; ++mm) {
      const int m = 2 * wave + mm;
      f32x4 ak[4], aw[4];
#pragma unroll
      for (int n = 0; n < 4; ++n) ak[n] = aw[n] = zero4();
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        const X8 a = ld8_tr(Ks, LDK, 32 * kb, 16 * m);
        const X8 w = fwt[mm][kb];
#pragma unroll
        for (int n = 0; n < 4; ++n) {
          if (n >= 2 * kb) ak[n] = mfma(a, ld8_tr(S1, LDT, 32 * kb, 16 * n), ak[n]);
          if (kb >= 1 || n < 2) {
            ak[n] = mfma(a, ld8(S1 + (16 * n + r) * LDT + 32 * kb + 8 * q4), ak[n]);
            aw[n] = mfma(w, ld8_tr(Ts, LDT, 32 * kb, 16 * n), aw[n]);
          }
        }
      }
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        const int t = 16 * n + r;
        const float bg = Bs[t] * __expf(Gs[t]);
        const f32x4 kk = krow[n][mm] = cvtf4(ld4(Ks + t * LDK + 16 * m + 4 * q4));
        // aw holds -(T^T dW): every use takes its sign back
        const float x = aw[n][0] * kk[0] + aw[n][1] * kk[1] + aw[n][2] * kk[2] + aw[n][3] * kk[3];
        colB[n] -= __expf(Gs[t]) * x;
        colG[n] -= bg * x;
        dkr[mm][n] = ak[n] + aw[n] * -bg + fkp[mm][n];
        pdk[n] += kk[0] * dkr[mm][n][0] + kk[1] * dkr[mm][n][1] + kk[2] * dkr[mm][n][2] + kk[3] * dkr[mm][n][3];
      }
    }
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      float xb = colB[n], xg = colG[n];
      xb = sum_rows4(xb);
      xg = sum_rows4(xg);
      if (q4 == 0) {
        dbl[16 * n + r] += xb;
        dgl[16 * n + r] += xg;
      }
    }
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      const float pd = sum_rows4(pdk[n]);
      if (q4 == 0) dkdot[4 * (16 * n + r) + wave] = pd;
    }
  }
  lds_barrier();

  // ---- wy phase 5: l2norm backward of dk; dg (reverse cumsum of the chunk's dG); dbeta ----
  const __amdgpu_buffer_rsrc_t dk_rs = chunk_rows_rsrc(dk, ci.start, ci.len, H, h);
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    const int t = 16 * n + r;
    const f32x4 d4 = *reinterpret_cast<const f32x4*>(&dkdot[4 * t]);
    const float dot = d4[0] + d4[1] + d4[2] + d4[3];
#pragma unroll
    for (int mm = 0; mm < 2; ++mm) {
      const int m = 2 * wave + mm;
      const f32x4 out = normalize ? (dkr[mm][n] - krow[n][mm] * dot) * rsn[n] : dkr[mm][n];
      buf_st4<E>(dk_rs, r * rowb + (16 * m + 4 * q4) * 2, 16 * n * rowb, F16 ? out * inv_dv : out);  // row t
    }
  }
  if (tid < 64) {
    const int t = tid;
    const bool in = t < ci.len;
    float x = keep_if(in, dgp_t + dgw[0][t] + dgw[1][t] + dgw[2][t] + dgw[3][t]);
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float o = __shfl_down(x, off, 64);
      if (t + off < 64) x += o;
    }
    if (in) {
      const float db = dbw[t] + dbw[64 + t] + dbw[128 + t] + dbw[192 + t];
      dg[(size_t)(ci.start + t) * H + h] = F16 ? x * inv_dv : x;
      dbeta[(size_t)(ci.start + t) * H + h] = F16 ? db * inv_dv : db;
    }
  }
}

// ---------------------------------------------------------------------------
// One wave on bwd_dkw's stream that ends once every reverse-scan workgroup has
// started (each adds one to *resident), so that bwd_dkw, launched behind it, can
// only take the CUs the scan leaves free and never holds one a scan workgroup
// still waits for.  Bounded: after COUNT_SPIN_LIMIT polls it ends anyway, and
// bwd_dkw's own bounded waits then decide.
__global__ __launch_bounds__(64) void scan_resident_gate_kernel(const int* __restrict__ resident, int expected) {
  if (threadIdx.x == 0) count_wait_ge<4>(resident, expected, COUNT_SPIN_LIMIT * 4);  // one wave: polls fast
}

static void launch_resident_gate(const int* resident, int expected, hipStream_t stream) {
  hipLaunchKernelGGL(scan_resident_gate_kernel, dim3(1), dim3(64), 0, stream, resident, expected);
}

// The scale target of dO: max|dO s_d| < 2^e with T 2^e <= 2^15, at most 2^1.
static int dout_scale_target(int T) {
  int lg = 0;
  while (lg < 31 && (1LL << lg) < (long long)T) ++lg;  // 2^lg >= T
  return 15 - lg < 1 ? 15 - lg : 1;
}

template <class E>
static hipError_t launch_bwd_t(const BwdArgs& a, hipStream_t stream) {
  auto F = [&](int i) { return reinterpret_cast<const E*>(a.fws + a.foff[i]); };
  auto Ff = [&](int i) { return reinterpret_cast<const float*>(a.fws + a.foff[i]); };
  auto B = [&](int i) { return reinterpret_cast<E*>(a.bws + a.boff[i]); };
  const E* q = static_cast<const E*>(a.q);
  const E* k = static_cast<const E*>(a.k);
  const E* v = static_cast<const E*>(a.v);
  const E* dout = static_cast<const E*>(a.dout);
  E* dq = static_cast<E*>(a.dq);
  E* dk = static_cast<E*>(a.dk);
  E* dv = static_cast<E*>(a.dv);
  const dim3 grid_p(a.H, a.n_chunks);  // chunk-major dispatch (the kernels pick the chunk order)
  int* sync = reinterpret_cast<int*>(a.bws + a.boff[B_SYNC]);
  int* ready = sync;                                 // [NC][H]
  int* resident = sync + (size_t)a.n_chunks * a.H;  // one count
  const bool beside = a.side != nullptr;
  // fp16: the scales s_d (partial maxima here, the scale itself in bwd_local) and s_v (the forward's)
  float* dsc = nullptr;
  const float* vsc = nullptr;
  if (__is_same(E, f16)) {
    dsc = reinterpret_cast<float*>(a.bws + a.boff[B_DSC]);
    vsc = Ff(F_VSC);
    launch_range_partials(a.dout, true, (size_t)a.T * a.H * (D / 8), nullptr, 0, dsc, stream);
  }
  {
    TimedLaunch tl(K_BWD_LOCAL, stream);
    hipLaunchKernelGGL(bwd_local_kernel<E>, dim3(a.H, a.n_chunks), dim3(256), 0, stream, q, k, (int)a.normalize, Ff(F_RK),
                       dout, Ff(F_GC), a.beta, F(F_TM), a.chunks, a.H, a.scale, dsc, dout_scale_target(a.T), B(B_DVLT),
                       B(B_XT), B(B_KNP), B(B_WT), sync);
  }
  if (beside) {
    if (const hipError_t e = hipEventRecord(a.side_fork, stream)) return e;
    if (const hipError_t e = hipStreamWaitEvent(a.side, a.side_fork, 0)) return e;
  }
  {
    TimedLaunch tl(K_BWD_SCAN, stream);
    hipLaunchKernelGGL(bwd_scan_kernel<E>, dim3(a.H * (D / 16), a.n_docs), dim3(BS_THREADS), 0, stream, B(B_KNP),
                       Ff(F_GC), B(B_DVLT), B(B_XT), B(B_WT), a.chunks, a.doc_chunk, a.H, B(B_DH), B(B_DVN),
                       beside ? ready : nullptr, beside ? resident : nullptr);
  }
  if (beside) {
    launch_resident_gate(resident, a.H * (D / 16) * a.n_docs, a.side);
    {
      TimedLaunch tl(K_BWD_DKW, a.side);
      hipLaunchKernelGGL(bwd_dkw_kernel<E>, grid_p, dim3(256), 0, a.side, q, k, Ff(F_RK), Ff(F_GC),
                         F(F_HT), F(F_VNT), dout, B(B_DH), B(B_DVN), v, a.beta, F(F_TM), a.chunks, a.H, a.scale,
                         (int)a.normalize, (const float*)dsc, vsc, dq, dk, dv, a.dg, a.dbeta, (const int*)ready,
                         a.dkw_never_ready ? D / 16 + 1 : D / 16, a.dkw_never_ready ? 4 : COUNT_SPIN_LIMIT);
    }
    if (const hipError_t e = hipEventRecord(a.side_join, a.side)) return e;
    return hipStreamWaitEvent(stream, a.side_join, 0);
  }
  if (a.dkw_after)
    if (const hipError_t e = hipStreamWaitEvent(stream, a.dkw_after, 0)) return e;
  TimedLaunch tl(K_BWD_DKW, stream);
  hipLaunchKernelGGL(bwd_dkw_kernel<E>, grid_p, dim3(256), 0, stream, q, k, Ff(F_RK), Ff(F_GC), F(F_HT),
                     F(F_VNT), dout, B(B_DH), B(B_DVN), v, a.beta, F(F_TM), a.chunks, a.H, a.scale, (int)a.normalize,
                     (const float*)dsc, vsc, dq, dk, dv, a.dg, a.dbeta, (const int*)nullptr, 0, 0);
  return hipSuccess;
}

hipError_t launch_bwd(const BwdArgs& a, hipStream_t stream) {
  return a.fp16 ? launch_bwd_t<f16>(a, stream) : launch_bwd_t<bf16>(a, stream);
}

}  // namespace cqgdn
