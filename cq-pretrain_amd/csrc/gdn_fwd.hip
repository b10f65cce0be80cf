// GDN forward on gfx950: chunk preparation, inter-chunk state scan, output.
//
// Math (per document, chunks of C = 64 events, state S in R^{K x V} fp32):
//   G = chunk-local cumsum(g), gam = exp(G), Gam_ij = exp(G_i - G_j) (i >= j)
//   A = strict_lower(beta_i * (k_i . k_j) * Gam_ij),  T = (I + A)^-1
//   W = T (beta*gam*K),  U = T (beta*V)
//   Vn = U - W S,  O = scale * [ (gam*Q) S + ((Q K^T) * Gam) Vn ]
//   S <- exp(G_last) S + (K * exp(G_last - G))^T Vn
// (reference_modeling_qwen3_5.py:344-411; the reference's op chain is the
//  K-b..K-g set of ops/gated_delta_net.py:144-183).
//
// Kernels:
//   fwd_prep   grid (NC, H), 4 waves: l2norm q,k; cumsum g; A via MFMA; the unit
//              lower-triangular inverse in LDS (fp32); W, W^T, U via MFMA.
//   fwd_state  grid (H * 8 value slices, docs), 1 wave: the serial scan, a 128x16
//              fp32 state slice held in registers across all chunks of a document.
//   fwd_out    grid (NC, H), 4 waves: O^T = gam * (h^T Qn^T) + Vn^T P^T, all MFMA.
#include "gdn_common.hpp"
#include "gdn_layout.hpp"
#include "gdn_kernels.hpp"

namespace cqgdn {

constexpr int LDK = 136;  // row stride (elements) of 64 x 128 tiles in LDS
constexpr int LDT = 72;   // row stride (elements) of 128 x 64 and 64 x 64 tiles in LDS
constexpr int LDA = 65;   // row stride (fp32) of the 64 x 64 solve matrix

// ---------------------------------------------------------------------------
// fwd_prep
// ---------------------------------------------------------------------------
// I: input element type of q, k, v (bf16 or f16).  E: operand element type (bf16,
// or f16 for the precise forward and for fp16 inputs).  vscale: with f16 operands,
// the power-of-two factor applied to V (fp16 range), which this kernel forms from
// the partial maxima after vscale[0] (range_scale, target vs_target) and stores in
// vscale[0] for the scan and the output kernel; null with bf16 operands.
template <class I, class E, bool NORMALIZE>
__global__ __launch_bounds__(256, 3) void fwd_prep_kernel(
    const I* __restrict__ k, const I* __restrict__ v,
    const float* __restrict__ g, const float* __restrict__ beta, const int32_t* __restrict__ chunks,
    int H, float* __restrict__ vscale, int vs_target,
    float* __restrict__ rk, float* __restrict__ gc, E* __restrict__ Tm, E* __restrict__ W,
    E* __restrict__ UT, E* __restrict__ KgT) {
  typedef typename Vec<E>::x8 X8;
  typedef typename Vec<E>::x4 X4;
  // grid (H, NC), chunks dispatched last to first: the state scan reads the
  // first chunks first, and they are then the most recently written (still in
  // the memory-side cache)
  const HeadChunk hc = xcd_head_chunk(gridDim.x, gridDim.y);  // all heads of a chunk on one XCD
  const int h = hc.h, c = gridDim.y - 1 - hc.p;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, q4 = lane >> 4;
  const ChunkInfo ci = chunk_info(chunks, c);
  const size_t cb = (size_t)c * H + h;

  __shared__ __attribute__((aligned(16))) float Gs[64];
  __shared__ __attribute__((aligned(16))) float Bs[64];
  __shared__ __attribute__((aligned(16))) E Ks[64 * LDK];      // K rows, then (beta gam K) rows
  __shared__ __attribute__((aligned(16))) float Af[64 * LDA];  // the solve's matrix, then the KgT tile
  __shared__ __attribute__((aligned(16))) E Ts[64 * LDT];
  __shared__ float red[4];
  // fp16 operands (the only ones with a scale): this thread's partial maximum of
  // |V|, requested before the other loads
  constexpr bool SCALED = __is_same(E, f16);
  const float vpart = SCALED ? range_partial4(vscale + 1) : 0.f;

  // Every global load is issued first, before any store (a wait for a load
  // also waits for every store issued before it), so the kernel pays one memory
  // round trip: the gates (wave 0), this thread's pieces of its k row,
  // and this wave's operand fragments of V for U = T (beta V), column gathers
  // for value tiles 2 wave, 2 wave + 1 (rows past the chunk re-read its last
  // row; their beta is zero).  Each phase waits only for what it reads: the
  // gathers' lane exchange runs where U is formed, and the stores of the row
  // phase go through buffer resources (rows past the chunk dropped by the range
  // check), so no store is conditional and the compiler can count what is in flight.
  // k is loaded non-temporally: nothing reads it again before the state scan,
  // whose operands (written here) then keep more of the memory-side cache.  q is
  // not read here: its l2 scale is formed by each kernel that reads q (row_rnorm).
  // (V's column gathers share lines between lanes and stay ordinary loads.)
  const int t_r = tid >> 2, p_r = tid & 3;  // row phase: thread (t, p) owns columns 8p + 32j, j = 0..3
  const size_t row_r = ((size_t)(ci.start + clamp_row(t_r, ci.len)) * H + h) * D;
  float gv = 0.f, bv = 0.f;
  if (wave == 0) {
    const size_t ev = (size_t)(ci.start + clamp_row(lane, ci.len)) * H + h;
    gv = g[ev];
    bv = beta[ev];
  }
  typename Vec<I>::x8 lk[4];
  Col8 vg[2][2];
#pragma unroll
  for (int j = 0; j < 4; ++j) lk[j] = ld8_nt(k + row_r + 32 * j + 8 * p_r);
  {
    const I* vb = v + ((size_t)ci.start * H + h) * D;
#pragma unroll
    for (int nn = 0; nn < 2; ++nn)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) vg[nn][kb] = col8_load_rows(vb, H * D, 32 * kb, 16 * (2 * wave + nn), ci.len);
  }
  // the scale of V, while the loads above are in flight (stored for the kernels
  // after this one at the end, where the store holds up no wait for a load)
  float vs = 1.f;
  if constexpr (SCALED) vs = range_scale(vpart, vs_target, red);
  const int rowe = H * D * (int)sizeof(E);  // bytes per event row of W
  const int rows_bytes = ((ci.len - 1) * H + 1) * D * (int)sizeof(E);
  const int gate_bytes = ((ci.len - 1) * H + 1) * (int)sizeof(float);

  // ---- gates: chunk-local cumsum of g (wave 0, one event per lane) ----
  if (wave == 0) {
    const bool in = lane < ci.len;
    gv = keep_if(in, gv);
    bv = keep_if(in, bv);
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float o = __shfl_up(gv, off, 64);
      if (lane >= off) gv += o;
    }
    Gs[lane] = gv;
    Bs[lane] = bv;
    buf_stf(buf_rsrc(gc + (size_t)ci.start * H + h, gate_bytes), lane * H * 4, 0, gv);  // rows past the chunk dropped
  }
  __syncthreads();
  const float glast = Gs[ci.len - 1];

  // ---- rows ----
  // Kg = K exp(G_last - G) is kept in registers and leaves through LDS after the
  // solve (coalesced rows of KgT instead of 2-byte scattered stores); beta gam K
  // (rounded once, from fp32) replaces K in LDS once A has been formed.
  X8 kg8[4], kb8[4];
  {
    const int t = t_r, p = p_r;
    const bool in = t < ci.len;
    const float gam_t = __expf(Gs[t]);
    const float kdec_t = __expf(glast - Gs[t]);
    const float b_t = Bs[t];
    const __amdgpu_buffer_rsrc_t rk_rs = buf_rsrc(rk + (size_t)ci.start * H + h, gate_bytes);
    // k
    {
      f32x8 x[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) x[j] = keep_if(in, cvtf8(lk[j]));
      float rs = 1.f;
      if (NORMALIZE) {
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int s = 0; s < 8; ++s) ss += x[j][s] * x[j][s];
        ss = sum4(ss);
        rs = rsqrtf(ss + 1e-6f);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f32x8 xn = x[j] * rs;
        const X8 xb = to8<E>(xn);
        const int col = 32 * j + 8 * p;
        st8(Ks + t * LDK + col, xb);
        kb8[j] = to8<E>(xn * (b_t * gam_t));
        kg8[j] = to8<E>(xn * kdec_t);
      }
      buf_stf(rk_rs, t * H * 4, 0, rs);
    }
  }
  __syncthreads();

  // ---- A = strict_lower(beta_t (k_t . k_s) Gam_ts): t-tile = wave, s-tiles <= wave ----
  {
    f32x4 acc[4];
#pragma unroll
    for (int n = 0; n < 4; ++n) acc[n] = zero4();
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const X8 a = ld8(Ks + (16 * wave + r) * LDK + 32 * kb + 8 * q4);
#pragma unroll
      for (int n = 0; n < 4; ++n)
        if (n <= wave) acc[n] = mfma(a, ld8(Ks + (16 * n + r) * LDK + 32 * kb + 8 * q4), acc[n]);
    }
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      const int s = 16 * n + r;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int t = 16 * wave + 4 * q4 + i;
        Af[t * LDA + s] = (s < t) ? Bs[t] * acc[n][i] * __expf(Gs[t] - Gs[s]) : 0.f;
      }
    }
  }
  __syncthreads();
  // every read of K is done: beta gam K takes its rows (read again only after the solve)
#pragma unroll
  for (int j = 0; j < 4; ++j) st8(Ks + t_r * LDK + 32 * j + 8 * p_r, kb8[j]);

  // ---- T = (I + A)^-1, blocked by 16, in fp32 ----
  // The four diagonal blocks by forward substitution (column c = tid/4 of block
  // c/16, lanes p split the sums), then the blocks below the diagonal level by
  // level (i - j = 1, 2, 3):  X_ij = sum_{k=j}^{i-1} A_ik T_kj,  T_ij = -T_ii X_ij.
  // Af then holds T_ii in the diagonal blocks and T_ij^T (i > j) in block
  // (j, i) above the diagonal (A's upper triangle is zero and unused); the
  // blocks below the diagonal still hold A.
  {
    const int col = tid >> 2, p = tid & 3, b0 = col & ~15, lc = col & 15;
    float tc[4];  // T[b0 + 4 jj + p][col]
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) tc[jj] = (4 * jj + p == lc) ? 1.f : 0.f;
#pragma unroll
    for (int i = 1; i < 16; ++i) {
      float part = 0.f;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) part += Af[(b0 + i) * LDA + b0 + 4 * jj + p] * tc[jj];
      part = sum4(part);
      const float val = (i > lc) ? -part : ((i == lc) ? 1.f : 0.f);
      if ((i & 3) == p) tc[i >> 2] = val;
    }
    __syncthreads();  // every read of A's diagonal blocks is done
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) Af[(b0 + 4 * jj + p) * LDA + col] = tc[jj];
  }
  // The levels below the diagonal, d = 1, 2, 3, on fp32 MFMA (16x16x4): wave w <
  // 4 - d owns the target block (ib, jb) = (w + d, w).  X = sum_{k=jb}^{ib-1}
  // A_{ib,k} T_{k,jb} reads only lower levels (T_{jb,jb} in its diagonal block,
  // T_{k,jb}, k > jb, transposed in block (jb, k)); X goes to the wave's own
  // block (jb, ib), transposed, and comes back as the operand of T_{ib,jb} =
  // -T_{ib,ib} X, which replaces it.  The block is the wave's alone (its LDS
  // operations complete in order), so the levels need one barrier each.
#pragma unroll
  for (int d = 1; d < 4; ++d) {
    __syncthreads();  // the diagonal blocks and the lower levels are complete
    if (wave < 4 - d) {
      const int jb = wave, ib = wave + d;
      const float* arow = Af + (16 * ib + r) * LDA + q4;  // A_{ib, .} row r at this lane's k (4 kk + q4)
      f32x4 x = zero4();
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
        x = mfma4(arow[16 * jb + 4 * kk], Af[(16 * jb + 4 * kk + q4) * LDA + 16 * jb + r], x);
      for (int kb = jb + 1; kb < ib; ++kb)
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
          x = mfma4(arow[16 * kb + 4 * kk], Af[(16 * jb + r) * LDA + 16 * kb + 4 * kk + q4], x);
      float* blk = Af + (16 * jb + r) * LDA + 16 * ib;  // block (jb, ib), row r: X^T, then T_{ib,jb}^T
#pragma unroll
      for (int i = 0; i < 4; ++i) blk[4 * q4 + i] = x[i];
      const float* trow = Af + (16 * ib + r) * LDA + 16 * ib + q4;  // T_{ib,ib} row r at k = 4 kk + q4
      f32x4 y = zero4();
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) y = mfma4(trow[4 * kk], blk[4 * kk + q4], y);
#pragma unroll
      for (int i = 0; i < 4; ++i) blk[4 * q4 + i] = -y[i];
    }
  }
  __syncthreads();
  {
    // T in the operand type: Ts rows [t][s], then the global copy from those rows.
    // The lanes of a wave run along one row (rows 4 jj + wave), so every read and
    // write of the copy touches 32 distinct banks (the solve matrix's row stride
    // is 65 words: its transposed blocks are read down consecutive rows).
    const int col = tid & 63, bcb = col >> 4;
#pragma unroll
    for (int jj = 0; jj < 16; ++jj) {
      const int t = 4 * jj + wave, bt = t >> 4;
      const float val = (bt == bcb) ? Af[t * LDA + col]
                                    : (bt > bcb ? Af[(16 * bcb + (col & 15)) * LDA + 16 * bt + (t & 15)] : 0.f);
      Ts[t * LDT + col] = (E)val;
    }
  }
  __syncthreads();
  {
    E* tm = Tm + cb * (CH * CH);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int seg = 256 * i + tid, row = seg >> 3, part = seg & 7;
      st8(tm + row * CH + 8 * part, ld8(Ts + row * LDT + 8 * part));
    }
  }

  // Kg^T tile [k][perm32(t)] over the solve's matrix (free now), stored below.
  // Row k's columns are XORed with 16 ((k / 8) % 4) (16-byte blocks stay whole):
  // the four threads of event t write rows 8 apart, which then fall in disjoint
  // banks instead of one.
  E* kgs = reinterpret_cast<E*>(Af);
  static_assert(sizeof(Af) >= D * CH * sizeof(E), "the KgT tile must fit the solve matrix");
  {
    const int t = tid >> 2, p = tid & 3, tp = perm32(t) ^ (16 * p);  // (k / 8) % 4 = p for k = 32 j + 8 p + s
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int s = 0; s < 8; ++s) kgs[(32 * j + 8 * p + s) * CH + tp] = kg8[j][s];
  }

  // ---- W = T (beta gam K) -> W rows, U = T (beta V) -> U^T storage ----
  // beta gam K is read transposed from its rows (ld8_tr); beta V comes from the
  // V fragments gathered at the start, scaled here.  (-W^T, the reverse scan's
  // operand, is formed by bwd_local.)
  {
    // U^T rows v = 16 (2 wave + nn) + 4 q4 .., all t tiles
    X8 bvf[2][2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const f32x4 b0 = *reinterpret_cast<const f32x4*>(Bs + 32 * kb + 8 * q4);
      const f32x4 b1 = *reinterpret_cast<const f32x4*>(Bs + 32 * kb + 8 * q4 + 4);
      const f32x8 bb = f32x8{b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]} * vs;
#pragma unroll
      for (int nn = 0; nn < 2; ++nn) bvf[nn][kb] = to8<E>(cvtf8(col8_combine_v<I>(vg[nn][kb])) * bb);
    }
    E* ut = UT + cb * (D * CH);
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      X8 a[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) a[kb] = ld8(Ts + (16 * tt + r) * LDT + 32 * kb + 8 * q4);
#pragma unroll
      for (int nn = 0; nn < 2; ++nn) {
        f32x4 au = zero4();
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
          if (kb == 0 || tt >= 2) au = mfma(a[kb], bvf[nn][kb], au);  // T[t][s] = 0 for s > t
        st4(ut + (16 * (2 * wave + nn) + r) * CH + 16 * tt + 4 * q4, au);
      }
    }
    const __amdgpu_buffer_rsrc_t w_rs = buf_rsrc(W + ((size_t)ci.start * H + h) * D, rows_bytes);
#pragma unroll
    for (int mm = 0; mm < 2; ++mm) {
      const int m = 2 * wave + mm;
      X8 ak[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) ak[kb] = ld8_trv<E>(Ks, LDK, 32 * kb, 16 * m);
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        f32x4 acc = zero4();
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) acc = mfma(ak[kb], ld8(Ts + (16 * n + r) * LDT + 32 * kb + 8 * q4), acc);
        // row t = 16 n + r (rows past the chunk fall outside w_rs)
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, to4<E>(-acc)), w_rs,
                                              r * rowe + perm32(16 * m + 4 * q4) * (int)sizeof(E), 16 * n * rowe, 0);
      }
    }
  }
  __syncthreads();
  {
    E* kgt = KgT + cb * (D * CH);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int seg = 256 * i + tid, kr = seg >> 3, part = seg & 7;
      st8(kgt + kr * CH + 8 * part, ld8(kgs + kr * CH + 8 * (part ^ (2 * ((kr >> 3) & 3)))));
    }
  }
  if (SCALED && blockIdx.x == 0 && blockIdx.y == 0 && tid == 0) vscale[0] = vs;
}

// ---------------------------------------------------------------------------
// fwd_state: one wave per (head, 16-wide value slice, document)
// ---------------------------------------------------------------------------
// The scan is a chain of dependent chunk steps, so it runs at the speed one
// step waits.  A workgroup serves one 16-wide value slice of one head with one
// consumer wave (wave 0) and two loader waves.  Loaders copy each chunk's
// operands global -> LDS asynchronously (global_load_lds) into a ring of
// SC_STAGES stages.  Each chunk's copies are split between the two loaders
// (issuing them is what bounds a step: a CU accepts about one 1 KB copy per
// 20-30 cycles, so one wave issuing all 35 takes longer than the consumer's
// MFMA work).  The consumer only reads LDS and writes its output tiles to LDS;
// loader 1 stores them.  So no wave holds in-flight data in registers and the
// consumer never waits on memory.
//
// The waves hand stages to each other through counts in LDS, not s_barrier:
// a loader publishes a chunk once its part has landed, the consumer publishes
// a chunk once it is done with it, and each wave waits only for the count it
// needs.  With a barrier per step, every step lasted as long as the slower of
// the consumer and the loaders plus the barrier; this way the loaders run up
// to four chunks ahead and the two sides overlap.
//
// LDS tiles are stored with 16-byte columns XOR-swizzled by row (chosen on the
// source side of each copy), so the consumer's fragment reads, 16 rows at one
// logical column, hit distinct banks:
//   W   [64 rows t][16 cols]  col' = col ^ (t & 15)
//   KgT [128 rows k][8 cols]  col' = col ^ ((k >> 1) & 7)
//   U^T [16 rows v][8 cols]   col' = col ^ ((v >> 1) & 7)
constexpr int SC_THREADS = 64 * 3;
constexpr int SC_STAGES = 4;
constexpr int SC_SROW = 136;  // scratch row stride (elements), S^T [v][k]
constexpr int SC_VROW = 72;   // scratch row stride (elements), v_new^T [v][t]

template <class E>
struct __attribute__((aligned(16))) FwdStage {
  E w[64 * 128];   // -W rows t
  E kg[128 * 64];  // KgT rows k
  E ut[16 * 64];   // U^T rows of the slice
  float glast;     // G of the chunk's last event
  float pad[3];
};

// the consumer's output tiles of a step, placed over the stage's KgT region
// once the consumer has read it (loader 1, which refills that region, stores
// them first)
template <class E>
struct __attribute__((aligned(16))) FwdScratch {
  E s[16 * SC_SROW];  // state entering the chunk, [v][k]
  E v[16 * SC_VROW];  // v_new, [v][t]
};
static_assert(sizeof(FwdScratch<bf16>) <= 128 * 64 * sizeof(bf16), "scratch must fit the KgT region");
template <class E>
__device__ __forceinline__ FwdScratch<E>& fwd_scratch(FwdStage<E>& st) {
  return *reinterpret_cast<FwdScratch<E>*>(st.kg);
}

// Per-lane byte offsets of a loader's copies within a full chunk (the same for
// every chunk of 64 events): part 0 the 16 W-row copies (from the chunk's first
// event row), part 1 the 16 KgT copies and the 2 U^T copies (from the chunk's
// tiles).  With them a full chunk's copy costs one address add.
template <int PART>
struct FwdCopyOffsets {
  uint32_t o[PART == 0 ? 16 : 18];
};
template <class E, int PART>
__device__ __forceinline__ FwdCopyOffsets<PART> fwd_copy_offsets(int H, int h, int lane) {
  FwdCopyOffsets<PART> f;
  if constexpr (PART == 0) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int t = 4 * i + (lane >> 4), col = (lane & 15) ^ (t & 15);
      f.o[i] = (uint32_t)(((t * H + h) * D + 8 * col) * sizeof(E));
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int k = 8 * i + (lane >> 3), col = (lane & 7) ^ ((k >> 1) & 7);
      f.o[i] = (uint32_t)((k * CH + 8 * col) * sizeof(E));
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int v = 8 * i + (lane >> 3), col = (lane & 7) ^ ((v >> 1) & 7);
      f.o[16 + i] = (uint32_t)((v * CH + 8 * col) * sizeof(E));
    }
  }
  return f;
}

// Issue the asynchronous copies of chunk c into stage S, in two parts: part 0
// (loader 0) the -W rows and G_last, 17 copies; part 1 (loader 1) KgT and the
// U^T slice, 18 copies.  Nothing here waits on memory: the chunk table is read
// with scalar loads and even the gate value travels by copy (a vector load
// whose result were used here would make this wave wait for every copy issued
// before it).  A tail chunk re-reads its last W row for the rows past its
// length (zeroed by fwd_fix_tail).
constexpr int FWD_PART_COPIES[2] = {17, 18};
template <class E, int PART>
__device__ __forceinline__ void fwd_issue(FwdStage<E>& S, const int32_t* __restrict__ chunks, int c, int H, int h,
                                          int v0, int lane, const FwdCopyOffsets<PART>& f,
                                          const E* __restrict__ W, const E* __restrict__ UT,
                                          const E* __restrict__ KgT, const float* __restrict__ gc) {
  const ChunkInfo ci = chunk_info(chunks, c);
  const size_t cb = (size_t)c * H + h;
  if constexpr (PART == 0) {
    if (ci.len == CH) {
      const char* base = reinterpret_cast<const char*>(W + (size_t)ci.start * H * D);
#pragma unroll
      for (int i = 0; i < 16; ++i) dma16(base + f.o[i], S.w + 512 * i);
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int t = 4 * i + (lane >> 4), col = (lane & 15) ^ (t & 15);
        const int tt = min(t, ci.len - 1);
        dma16(W + ((size_t)(ci.start + tt) * H + h) * D + 8 * col, S.w + 512 * i);
      }
    }
    if (lane == 0)  // one lane: a dword copy writes 4 bytes per active lane
      __builtin_amdgcn_global_load_lds(gc + (size_t)(ci.start + ci.len - 1) * H + h, (lds_void_ptr)&S.glast, 4, 0,
                                       0);
  } else {
    const char* kg = reinterpret_cast<const char*>(KgT + cb * (D * CH));
#pragma unroll
    for (int i = 0; i < 16; ++i) dma16(kg + f.o[i], S.kg + 512 * i);
    const char* ut = reinterpret_cast<const char*>(UT + cb * (D * CH) + v0 * CH);
#pragma unroll
    for (int i = 0; i < 2; ++i) dma16(ut + f.o[16 + i], S.ut + 512 * i);
  }
}

// After the copies of chunk c have landed: zero the W rows past its length.
template <class E>
__device__ __forceinline__ void fwd_fix_tail(FwdStage<E>& S, const int32_t* __restrict__ chunks, int c, int lane) {
  const int len = chunk_info(chunks, c).len;
  if (len < CH) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int t = 4 * i + (lane >> 4);
      if (t >= len) st8(S.w + t * 128 + 8 * (lane & 15), zero8v<E>());
    }
  }
}

// global stores of one copy-out (4 of h^T, 2 of v_new^T)
constexpr int FWD_OUT_STORES = 6;

// scratch of one step -> hT [v0..v0+15][k], vnT [v0..v0+15][t]; NaN instead once
// a hand-off wait has given up (the scratch may then hold another step's values)
template <class E>
__device__ __forceinline__ void fwd_copy_out(const FwdScratch<E>& sc, int c, int H, int h, int v0, int lane,
                                             bool poison, E* __restrict__ hT, E* __restrict__ vnT) {
  typedef typename Vec<E>::x8 X8;
  const size_t cb = (size_t)c * H + h;
  const X8 nan8 = to8<E>(f32x8{NAN, NAN, NAN, NAN, NAN, NAN, NAN, NAN});
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int seg = 64 * i + lane, v = seg >> 4, ks = seg & 15;
    const X8 x = ld8(sc.s + v * SC_SROW + 8 * ks);
    st8(hT + cb * (D * D) + (v0 + v) * D + 8 * ks, poison ? nan8 : x);
  }
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int seg = 64 * i + lane, v = seg >> 3, ts = seg & 7;
    const X8 x = ld8(sc.v + v * SC_VROW + 8 * ts);
    st8(vnT + cb * (D * CH) + (v0 + v) * CH + 8 * ts, poison ? nan8 : x);
  }
}

// Loader PART of the forward scan, iteration x: publish chunk x-2 as soon as
// this loader's part of it has landed, then, once the consumer is done with
// chunk x-4, refill that chunk's stage (x % 4) with this loader's part of
// chunk x (loader 1 first stores chunk x-4's outputs from the stage's KgT
// region).  Loads and stores retire in issue order (one counter on gfx9), so a
// loader waits for chunk x-2 by letting exactly the operations it issued after
// that part stay in flight: its part of chunk x-1 and, for loader 1, the
// copy-out before it.
template <class E, int PART>
__device__ __forceinline__ void fwd_loader(FwdStage<E>* stage, int* flags, const int32_t* __restrict__ chunks,
                                           int c_begin, int n, int H, int h, int v0, int lane,
                                           const E* __restrict__ W, const E* __restrict__ UT,
                                           const E* __restrict__ KgT, const float* __restrict__ gc,
                                           E* __restrict__ hT, E* __restrict__ vnT) {
  const FwdCopyOffsets<PART> offs = fwd_copy_offsets<E, PART>(H, h, lane);
  // Once a wait gives up, the rest run without waiting, and flags[3] tells the
  // consumer, which turns its state (and so every later output) to NaN: stages
  // refilled without the wait may be overwritten while it reads them.
  bool ok = true;
  for (int x = 0; x < n + SC_STAGES; ++x) {
    const int y = x - 2;
    if (y >= 0 && y < n) {
      const int parts = x - 1 < n;
      if constexpr (PART == 0) {
        wait_vmem_parts<FWD_PART_COPIES[0], FWD_OUT_STORES>(parts, 0);
        fwd_fix_tail(stage[y & (SC_STAGES - 1)], chunks, c_begin + y, lane);
      } else {
        wait_vmem_parts<FWD_PART_COPIES[1], FWD_OUT_STORES>(parts, x - 5 >= 0 && x - 5 < n);
      }
      lds_flag_publish(&flags[PART], y + 1);
    }
    if (x >= SC_STAGES) {
      if (ok) {
        ok = lds_flag_wait_ge<true>(&flags[2], x - SC_STAGES + 1);
        if (!ok) {  // published (and complete in LDS) before this wave refills any stage
          lds_flag_publish(&flags[3], 1);
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        }
      }
      if (PART == 1 && x - SC_STAGES < n)
        fwd_copy_out(fwd_scratch(stage[x & (SC_STAGES - 1)]), c_begin + x - SC_STAGES, H, h, v0, lane,
                     lds_flag_read(&flags[3]) != 0, hT, vnT);
    }
    if (x < n) fwd_issue<E, PART>(stage[x & (SC_STAGES - 1)], chunks, c_begin + x, H, h, v0, lane, offs, W, UT, KgT, gc);
  }
}

template <class E>
__global__ __launch_bounds__(SC_THREADS) void fwd_scan_kernel(
    const E* __restrict__ W, const E* __restrict__ UT, const E* __restrict__ KgT,
    const float* __restrict__ gc, const int32_t* __restrict__ chunks, const int32_t* __restrict__ doc_chunk,
    int H, const float* __restrict__ vscale, const float* __restrict__ init_state, float* __restrict__ final_state,
    E* __restrict__ hT, E* __restrict__ vnT) {
  typedef typename Vec<E>::x8 X8;
  typedef typename Vec<E>::x4 X4;
  // blockIdx.x = slice * H + h: the slices of one head land on one XCD when H % 8 == 0
  const int h = blockIdx.x % H, slice = blockIdx.x / H, d = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, q4 = lane >> 4;
  const int v0 = 16 * slice;

  __shared__ FwdStage<E> stage[SC_STAGES];
  // hand-off counts: [0], [1] chunks whose part from loader 0 / 1 has landed
  // (and, for loader 0, whose tail rows are zeroed); [2] chunks the consumer
  // has finished (operands read, outputs in the stage's scratch); [3] nonzero
  // once a loader's wait for the consumer has given up
  __shared__ __attribute__((aligned(16))) int flags[4];
  if (threadIdx.x < 4) flags[threadIdx.x] = 0;
  __syncthreads();

  const int c_begin = doc_chunk[d], n = doc_chunk[d + 1] - c_begin;
  if (wave == 0) {
    f32x4 S[8];  // S[m][i] = state[k = 16m + 4q4 + i][v = v0 + r]
#pragma unroll
    for (int m = 0; m < 8; ++m) S[m] = zero4();
    const float vs = vscale ? *vscale : 1.f;  // the state is carried in the scale of V
    if (init_state) {
      const float* s0 = init_state + ((size_t)d * H + h) * D * D;
#pragma unroll
      for (int m = 0; m < 8; ++m)
#pragma unroll
        for (int i = 0; i < 4; ++i) S[m][i] = s0[(16 * m + 4 * q4 + i) * D + v0 + r] * vs;
    }
    // per-lane parts of the swizzled LDS addresses (bytes); the row parts are
    // compile-time offsets of each read
    int wofs[4], kofs[2], uofs[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) wofs[j] = 2 * (r * 128 + 8 * ((4 * j + q4) ^ r));
#pragma unroll
    for (int j = 0; j < 2; ++j) kofs[j] = 2 * (r * 64 + 8 * ((4 * j + q4) ^ ((r >> 1) & 7)));
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) uofs[i4] = 2 * (r * 64 + 8 * ((2 * i4 + (q4 >> 1)) ^ ((r >> 1) & 7)) + 4 * (q4 & 1));
    const int sofs = 2 * (r * SC_SROW + 4 * q4), vofs = 2 * (r * SC_VROW + 4 * q4);
    int seen = 0;       // both loaders' counts are at least this (last read)
    bool ok = true;     // every hand-off wait succeeded
    int poisoned = 0;   // flags[3] as last read
    for (int tau = 0; tau < n; ++tau) {
      if (ok && seen <= tau) ok = scan_wait_ready(flags, tau + 1, seen);
      if (poisoned) ok = false;
      if (!ok) {  // a broken hand-off: make every later output NaN
        // (the empty asm keeps this a branch: as selects it cost 32 VALU operations a step)
        asm volatile("");
#pragma unroll
        for (int m = 0; m < 8; ++m) S[m] = f32x4{NAN, NAN, NAN, NAN};
      }
      char* base = reinterpret_cast<char*>(&stage[tau & (SC_STAGES - 1)]);
      const char* wb = base + offsetof(FwdStage<E>, w);
      const char* kb = base + offsetof(FwdStage<E>, kg);
      const char* ub = base + offsetof(FwdStage<E>, ut);
      // every operand read is issued ahead of the MFMAs that use them (the W
      // fragments first); the scheduling barriers keep the compiler from
      // interleaving them one by one
      X8 fw[4][4], fk[8][2];
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) fw[i4][j] = *reinterpret_cast<const X8*>(wb + wofs[j] + 4096 * i4);
      f32x4 vn[4];
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) vn[i4] = cvtf4(*reinterpret_cast<const X4*>(ub + uofs[i4]));
      const float glast = reinterpret_cast<const FwdStage<E>*>(base)->glast;
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int m = 0; m < 8; ++m) fk[m][j] = *reinterpret_cast<const X8*>(kb + kofs[j] + 2048 * m);
      const int2 pre = lds_flag_read2(flags);  // for the next step, read while this one computes
      poisoned = lds_flag_read(&flags[3]);
      __builtin_amdgcn_sched_barrier(0);
      X4 sh[8];
#pragma unroll
      for (int m = 0; m < 8; ++m) sh[m] = to4<E>(S[m]);
      // v_new = U + (-W) S; the state's decay runs beside it
      const float gC = __expf(glast);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const X8 hb = cat(sh[2 * j], sh[2 * j + 1]);
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) vn[i4] = mfma(fw[i4][j], hb, vn[i4]);
#pragma unroll
        for (int m = 2 * j; m < 2 * j + 2; ++m) S[m] *= gC;
      }
      __builtin_amdgcn_sched_barrier(0);
      // the KgT fragments have been read (a wave's LDS operations complete in
      // order): the KgT region now takes this step's outputs
      char* sb = base + offsetof(FwdStage<E>, kg);
#pragma unroll
      for (int m = 0; m < 8; ++m) *reinterpret_cast<X4*>(sb + sofs + 32 * m) = sh[m];
      // S <- exp(G_last) S + (K exp(G_last - G))^T v_new
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const X8 vb = pack_permv<E>(vn[2 * j], vn[2 * j + 1]);
#pragma unroll
        for (int m = 0; m < 8; ++m) S[m] = mfma(fk[m][j], vb, S[m]);
      }
      char* vbp = sb + sizeof(FwdScratch<E>::s);
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) *reinterpret_cast<X4*>(vbp + vofs + 32 * i4) = to4<E>(vn[i4]);
      lds_flag_publish(&flags[2], tau + 1);
      seen = max(seen, min(__builtin_amdgcn_readfirstlane(pre.x), __builtin_amdgcn_readfirstlane(pre.y)));
    }
    if (final_state) {
      float* sf = final_state + ((size_t)d * H + h) * D * D;
      const float inv = 1.f / vs;  // exact: vs is a power of two
#pragma unroll
      for (int m = 0; m < 8; ++m)
#pragma unroll
        for (int i = 0; i < 4; ++i) sf[(16 * m + 4 * q4 + i) * D + v0 + r] = S[m][i] * inv;
    }
  } else {
    // The loader's part is a template argument, so its copy offsets stay in
    // registers (indexed by a run-time part they went to scratch memory, and
    // reloading them waited for every copy in flight).
    if (wave == 1)
      fwd_loader<E, 0>(stage, flags, chunks, c_begin, n, H, h, v0, lane, W, UT, KgT, gc, hT, vnT);
    else
      fwd_loader<E, 1>(stage, flags, chunks, c_begin, n, H, h, v0, lane, W, UT, KgT, gc, hT, vnT);
  }
}

// ---------------------------------------------------------------------------
// fwd_out: O^T (v rows, t columns) per chunk and head.
// ---------------------------------------------------------------------------
template <class I, class E>  // I: element type of q, k and o; E: operand type (as fwd_prep)
__global__ __launch_bounds__(256) void fwd_out_kernel(
    const I* __restrict__ q, const I* __restrict__ k, int normalize,
    const float* __restrict__ rk, const float* __restrict__ gc, const E* __restrict__ hT,
    const E* __restrict__ vnT, const int32_t* __restrict__ chunks, int H,
    float scale, const float* __restrict__ vscale, I* __restrict__ o) {
  typedef typename Vec<E>::x8 X8;
  // grid (H, NC), chunks last to first: the state scan wrote the last chunks
  // last, so they are the likeliest still in the memory-side cache
  const HeadChunk hc = xcd_head_chunk(gridDim.x, gridDim.y);  // all heads of a chunk on one XCD
  const int h = hc.h, c = gridDim.y - 1 - hc.p;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, q4 = lane >> 4;
  const ChunkInfo ci = chunk_info(chunks, c);
  const size_t cb = (size_t)c * H + h;

  __shared__ __attribute__((aligned(16))) E Qs[64 * LDK];
  __shared__ __attribute__((aligned(16))) E Ks[64 * LDK];
  __shared__ __attribute__((aligned(16))) E Ps[64 * LDT];  // P[t][s], causal, gated
  __shared__ float Gs[64];

  const E* ht = hT + cb * (D * D);
  const E* vt = vnT + cb * (D * CH);
  // requested with the inputs: rows v = 16 (2 wave + mm) + r of v_new^T (t block
  // kb) and of h^T (k block kb)
  X8 av[2][2], ah[2][4];
#pragma unroll
  for (int mm = 0; mm < 2; ++mm) {
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) av[mm][kb] = ld8(vt + (16 * (2 * wave + mm) + r) * CH + 32 * kb + 8 * q4);
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) ah[mm][kb] = ld8(ht + (16 * (2 * wave + mm) + r) * D + 32 * kb + 8 * q4);
  }
  {
    const int t = tid >> 2, p = tid & 3;
    const bool in = t < ci.len;
    const size_t ev = (size_t)(ci.start + clamp_row(t, ci.len)) * H + h, row = ev * D;
    const float rkt = rk[ev];
    typename Vec<I>::x8 xq[4], xk[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int col = 32 * j + 8 * p;
      xq[j] = ld8(q + row + col);
      xk[j] = ld8(k + row + col);
    }
    if (p == 0) Gs[t] = gc[ev];
    const float rqt = normalize ? row_rnorm(xq) : 1.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int col = 32 * j + 8 * p;
      st8(Qs + t * LDK + col, keep_if(in, scaled8<E>(xq[j], rqt)));
      st8(Ks + t * LDK + col, keep_if(in, scaled8<E>(xk[j], rkt)));
    }
  }
  __syncthreads();

  // P^T tiles: s-tile a = wave, t-tiles b >= a
  {
    const int a = wave;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      f32x4 acc = zero4();
      if (b >= a) {
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
          acc = mfma(ld8(Ks + (16 * a + r) * LDK + 32 * kb + 8 * q4), ld8(Qs + (16 * b + r) * LDK + 32 * kb + 8 * q4),
                     acc);
        const int t = 16 * b + r;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int s = 16 * a + 4 * q4 + i;
          acc[i] = (s <= t) ? acc[i] * __expf(Gs[t] - Gs[s]) : 0.f;
        }
      }
      st4(Ps + (16 * b + r) * LDT + 16 * a + 4 * q4, acc);
    }
  }
  __syncthreads();

  // O^T = (h^T Qn^T) * gam_t + Vn^T P^T ; wave owns value tiles 2w, 2w+1
  f32x4 acc[2][4];
#pragma unroll
  for (int mm = 0; mm < 2; ++mm)
#pragma unroll
    for (int n = 0; n < 4; ++n) acc[mm][n] = zero4();
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    X8 bq[4];
#pragma unroll
    for (int n = 0; n < 4; ++n) bq[n] = ld8(Qs + (16 * n + r) * LDK + 32 * kb + 8 * q4);
#pragma unroll
    for (int mm = 0; mm < 2; ++mm)
#pragma unroll
      for (int n = 0; n < 4; ++n) acc[mm][n] = mfma(ah[mm][kb], bq[n], acc[mm][n]);
  }
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    const float gam = __expf(Gs[16 * n + r]);
#pragma unroll
    for (int mm = 0; mm < 2; ++mm) acc[mm][n] *= gam;
  }
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      if (n < 2 * kb) continue;  // t-tile n holds no s in this block (s > t)
      const X8 b = ld8(Ps + (16 * n + r) * LDT + 32 * kb + 8 * q4);
#pragma unroll
      for (int mm = 0; mm < 2; ++mm) acc[mm][n] = mfma(av[mm][kb], b, acc[mm][n]);
    }
  }
  const float osc = vscale ? scale / *vscale : scale;  // undo the power-of-two scale of V
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    const int t = 16 * n + r;
    if (t >= ci.len) continue;
    I* orow = o + ((size_t)(ci.start + t) * H + h) * D;
#pragma unroll
    for (int mm = 0; mm < 2; ++mm) st4(orow + 16 * (2 * wave + mm) + 4 * q4, acc[mm][n] * osc);
  }
}

// ---------------------------------------------------------------------------
// Power-of-two scale of V for the fp16 forwards.  The recurrence is linear in
// (V, initial state): scaling both by vs scales W-free quantities (U, v_new,
// every state, O) by vs exactly, so the kernels carry them scaled and divide O
// and the final state by vs.  vs brings max(|V|, |S0|) into [2^(t-1), 2^t):
// t = 6 for inference, far inside fp16's range (65504) for U, v_new and the
// state; t = 3 for training, where the backward multiplies V-scaled by
// dO-scaled quantities (dP, dW) and keeps their products in fp16 too.  The same
// kernels give the backward's scale of dO (launch_range_partials, then bwd_local).
// ---------------------------------------------------------------------------
constexpr int VS_BLOCKS = kVscaleBlocks;

__device__ __forceinline__ float block_max(float m, float* red) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

template <class I>
__global__ __launch_bounds__(256) void vscale_partial_kernel(const I* __restrict__ v, size_t nv8,
                                                             const float* __restrict__ s0, size_t ns,
                                                             float* __restrict__ part) {
  __shared__ float red[4];
  float m = 0.f;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  // eight 16-byte loads in flight per thread: one at a time, the loop waits out a
  // memory round trip per load and reads at about a quarter of HBM's rate
  // (the last round's loads past the end are skipped lane by lane, all in one round trip)
  constexpr int U = 8;
  for (; i < nv8; i += U * stride) {
    typename Vec<I>::x8 x[U];
#pragma unroll
    for (int u = 0; u < U; ++u) x[u] = i + u * stride < nv8 ? ld8(v + 8 * (i + u * stride)) : zero8v<I>();
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const f32x8 f = cvtf8(x[u]);
#pragma unroll
      for (int s = 0; s < 8; ++s) m = fmaxf(m, fabsf(f[s]));
    }
  }
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < ns; i += stride) m = fmaxf(m, fabsf(s0[i]));
  m = block_max(m, red);
  if (threadIdx.x == 0) part[blockIdx.x] = m;
}

// ---------------------------------------------------------------------------
// host launchers
// ---------------------------------------------------------------------------
template <class I, class E>
static hipError_t launch_fwd_t(const FwdArgs& a, float* vscale, int vs_target, hipStream_t stream) {
  E* ws[F_COUNT];
  for (int i = 0; i < F_COUNT; ++i) ws[i] = reinterpret_cast<E*>(a.ws + a.off[i]);
  float* rk = reinterpret_cast<float*>(ws[F_RK]);
  float* gcum = reinterpret_cast<float*>(ws[F_GC]);
  const I* q = static_cast<const I*>(a.q);
  const I* k = static_cast<const I*>(a.k);
  const I* v = static_cast<const I*>(a.v);
  {
    TimedLaunch tl(K_FWD_PREP, stream);
    const dim3 grid_p(a.H, a.n_chunks);
    if (a.normalize)
      hipLaunchKernelGGL((fwd_prep_kernel<I, E, true>), grid_p, dim3(256), 0, stream, k, v, a.g, a.beta,
                         a.chunks, a.H, vscale, vs_target, rk, gcum, ws[F_TM], ws[F_W],
                         ws[F_UT], ws[F_KGT]);
    else
      hipLaunchKernelGGL((fwd_prep_kernel<I, E, false>), grid_p, dim3(256), 0, stream, k, v, a.g, a.beta,
                         a.chunks, a.H, vscale, vs_target, rk, gcum, ws[F_TM], ws[F_W],
                         ws[F_UT], ws[F_KGT]);
  }
  const dim3 grid_s(a.H * (D / 16), a.n_docs);
  hipStream_t ss = stream;
  if (a.scan_stream) {
    if (const hipError_t e = hipEventRecord(a.scan_fork, stream)) return e;
    if (const hipError_t e = hipStreamWaitEvent(a.scan_stream, a.scan_fork, 0)) return e;
    ss = a.scan_stream;
  }
  {
    TimedLaunch tl(K_FWD_SCAN, ss);
    hipLaunchKernelGGL(fwd_scan_kernel<E>, grid_s, dim3(SC_THREADS), 0, ss, ws[F_W], ws[F_UT], ws[F_KGT], gcum,
                       a.chunks, a.doc_chunk, a.H, vscale, a.initial_state, a.final_state, ws[F_HT], ws[F_VNT]);
  }
  if (a.scan_stream)
    if (const hipError_t e = hipEventRecord(a.scan_join, a.scan_stream)) return e;
  if (a.no_output) return hipSuccess;
  TimedLaunch tl(K_FWD_OUT, stream);
  hipLaunchKernelGGL((fwd_out_kernel<I, E>), dim3(a.H, a.n_chunks), dim3(256), 0, stream, q, k, (int)a.normalize, rk, gcum,
                     ws[F_HT], ws[F_VNT], a.chunks, a.H, a.scale, vscale, static_cast<I*>(a.o));
  return hipSuccess;
}

void launch_range_partials(const void* x, bool fp16, size_t n8, const float* s0, size_t ns, float* out,
                           hipStream_t stream) {
  static_assert(VS_BLOCKS == 4 * 256, "range_partial4 takes four partials per thread of a 256-thread workgroup");
  if (fp16)
    hipLaunchKernelGGL(vscale_partial_kernel<f16>, dim3(VS_BLOCKS), dim3(256), 0, stream,
                       static_cast<const f16*>(x), n8, s0, ns, out + 1);
  else
    hipLaunchKernelGGL(vscale_partial_kernel<bf16>, dim3(VS_BLOCKS), dim3(256), 0, stream,
                       static_cast<const bf16*>(x), n8, s0, ns, out + 1);
}

hipError_t launch_fwd(const FwdArgs& a, hipStream_t stream) {
  if (!a.precise && !a.fp16) return launch_fwd_t<bf16, bf16>(a, nullptr, 0, stream);
  float* vsc = reinterpret_cast<float*>(a.ws + a.off[F_VSC]);
  const size_t nv8 = (size_t)a.T * a.H * (D / 8);
  const size_t ns = a.initial_state ? (size_t)a.n_docs * a.H * D * D : 0;
  launch_range_partials(a.v, a.fp16, nv8, a.initial_state, ns, vsc, stream);
  const int target = a.training ? kVscaleTargetTraining : kVscaleTarget;
  return a.fp16 ? launch_fwd_t<f16, f16>(a, vsc, target, stream) : launch_fwd_t<bf16, f16>(a, vsc, target, stream);
}

}  // namespace cqgdn
