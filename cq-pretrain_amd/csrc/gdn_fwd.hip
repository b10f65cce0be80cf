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

constexpr int LDK = 136;  // row stride (bf16) of 64 x 128 tiles in LDS
constexpr int LDT = 72;   // row stride (bf16) of 128 x 64 and 64 x 64 tiles in LDS
constexpr int LDA = 65;   // row stride (fp32) of the 64 x 64 solve matrix

// ---------------------------------------------------------------------------
// fwd_prep
// ---------------------------------------------------------------------------
template <bool NORMALIZE>
__global__ __launch_bounds__(256) void fwd_prep_kernel(
    const bf16* __restrict__ q, const bf16* __restrict__ k, const bf16* __restrict__ v,
    const float* __restrict__ g, const float* __restrict__ beta, const int32_t* __restrict__ chunks,
    int H, bf16* __restrict__ qn, bf16* __restrict__ kn, float* __restrict__ rq,
    float* __restrict__ rk, float* __restrict__ gc, bf16* __restrict__ Tm, bf16* __restrict__ W,
    bf16* __restrict__ WT, bf16* __restrict__ UT, bf16* __restrict__ KgT) {
  const int c = blockIdx.x, h = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, q4 = lane >> 4;
  const ChunkInfo ci = chunk_info(chunks, c);
  const size_t cb = (size_t)c * H + h;

  __shared__ float Gs[64], Bs[64];
  __shared__ __attribute__((aligned(16))) bf16 Ks[64 * LDK];
  __shared__ __attribute__((aligned(16))) bf16 KbT[128 * LDT];
  __shared__ __attribute__((aligned(16))) bf16 VbT[128 * LDT];
  __shared__ float Af[64 * LDA];
  __shared__ __attribute__((aligned(16))) bf16 Ts[64 * LDT];

  // ---- gates: chunk-local cumsum of g (wave 0, one event per lane) ----
  if (wave == 0) {
    const int t = lane;
    const bool in = t < ci.len;
    float gv = in ? g[(size_t)(ci.start + t) * H + h] : 0.f;
    const float bv = in ? beta[(size_t)(ci.start + t) * H + h] : 0.f;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float o = __shfl_up(gv, off, 64);
      if (lane >= off) gv += o;
    }
    Gs[t] = gv;
    Bs[t] = bv;
    if (in) gc[(size_t)(ci.start + t) * H + h] = gv;
  }
  __syncthreads();
  const float glast = Gs[ci.len - 1];

  // ---- rows: thread (t, p) owns columns 8p + 32j, j = 0..3 ----
  {
    const int t = tid >> 2, p = tid & 3;
    const bool in = t < ci.len;
    const size_t row = ((size_t)(ci.start + t) * H + h) * D;
    const float gam_t = __expf(Gs[t]);
    const float kdec_t = __expf(glast - Gs[t]);
    const float b_t = Bs[t];
    // q
    {
      f32x8 x[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) x[j] = in ? cvtf8(ld8(q + row + 32 * j + 8 * p)) : f32x8{};
      float rs = 1.f;
      if (NORMALIZE) {
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int s = 0; s < 8; ++s) ss += x[j][s] * x[j][s];
        ss += __shfl_xor(ss, 1, 64);
        ss += __shfl_xor(ss, 2, 64);
        rs = rsqrtf(ss + 1e-6f);
      }
      if (in) {
#pragma unroll
        for (int j = 0; j < 4; ++j) st8(qn + row + 32 * j + 8 * p, cvt8(x[j] * rs));
        if (p == 0) rq[(size_t)(ci.start + t) * H + h] = rs;
      }
    }
    // k
    {
      f32x8 x[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) x[j] = in ? cvtf8(ld8(k + row + 32 * j + 8 * p)) : f32x8{};
      float rs = 1.f;
      if (NORMALIZE) {
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int s = 0; s < 8; ++s) ss += x[j][s] * x[j][s];
        ss += __shfl_xor(ss, 1, 64);
        ss += __shfl_xor(ss, 2, 64);
        rs = rsqrtf(ss + 1e-6f);
      }
      bf16* kgt = KgT + cb * (D * CH);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const f32x8 xn = x[j] * rs;
        const bf16x8 xb = cvt8(xn);
        const int col = 32 * j + 8 * p;
        st8(Ks + t * LDK + col, xb);
        if (in) st8(kn + row + col, xb);
        const f32x8 xbg = xn * (b_t * gam_t);
        const f32x8 xkd = xn * kdec_t;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          KbT[(col + s) * LDT + t] = (bf16)xbg[s];
          kgt[(col + s) * CH + t] = (bf16)xkd[s];
        }
      }
      if (in && p == 0) rk[(size_t)(ci.start + t) * H + h] = rs;
    }
    // v
    {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int col = 32 * j + 8 * p;
        const f32x8 x = in ? cvtf8(ld8(v + row + col)) * b_t : f32x8{};
#pragma unroll
        for (int s = 0; s < 8; ++s) VbT[(col + s) * LDT + t] = (bf16)x[s];
      }
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
      const bf16x8 a = ld8(Ks + (16 * wave + r) * LDK + 32 * kb + 8 * q4);
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

  // ---- T = (I + A)^-1 by forward substitution: column c = tid/4, lanes p split the sum ----
  {
    const int col = tid >> 2, p = tid & 3;
    float tc[16];
#pragma unroll
    for (int jj = 0; jj < 16; ++jj) tc[jj] = (4 * jj + p == col) ? 1.f : 0.f;
#pragma unroll
    for (int i = 1; i < 64; ++i) {
      float part = 0.f;
#pragma unroll
      for (int jj = 0; jj <= (i - 1) / 4; ++jj) part += Af[i * LDA + 4 * jj + p] * tc[jj];
      part += __shfl_xor(part, 1, 64);
      part += __shfl_xor(part, 2, 64);
      const float val = (i > col) ? -part : ((i == col) ? 1.f : 0.f);
      if ((i & 3) == p) tc[i >> 2] = val;
    }
    bf16* tm = Tm + cb * (CH * CH);
#pragma unroll
    for (int jj = 0; jj < 16; ++jj) {
      const bf16 b = (bf16)tc[jj];
      Ts[(4 * jj + p) * LDT + col] = b;
      tm[(4 * jj + p) * CH + col] = b;
    }
  }
  __syncthreads();

  // ---- W (-> W^T storage), W^T (-> W rows), U (-> U^T storage) ----
  {
    bf16x8 at[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) at[kb] = ld8(Ts + (16 * wave + r) * LDT + 32 * kb + 8 * q4);
    bf16* wt = WT + cb * (D * CH);
    bf16* ut = UT + cb * (D * CH);
#pragma unroll
    for (int n = 0; n < 8; ++n) {
      f32x4 aw = zero4(), au = zero4();
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        aw = mfma(at[kb], ld8(KbT + (16 * n + r) * LDT + 32 * kb + 8 * q4), aw);
        au = mfma(at[kb], ld8(VbT + (16 * n + r) * LDT + 32 * kb + 8 * q4), au);
      }
      st4(wt + (16 * n + r) * CH + 16 * wave + 4 * q4, aw);
      st4(ut + (16 * n + r) * CH + 16 * wave + 4 * q4, au);
    }
#pragma unroll
    for (int mm = 0; mm < 2; ++mm) {
      const int m = 2 * wave + mm;
      bf16x8 ak[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) ak[kb] = ld8(KbT + (16 * m + r) * LDT + 32 * kb + 8 * q4);
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        f32x4 acc = zero4();
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) acc = mfma(ak[kb], ld8(Ts + (16 * n + r) * LDT + 32 * kb + 8 * q4), acc);
        const int t = 16 * n + r;
        if (t < ci.len) st4(W + ((size_t)(ci.start + t) * H + h) * D + 16 * m + 4 * q4, acc);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// fwd_state: one wave per (head, 16-wide value slice, document)
// ---------------------------------------------------------------------------
template <bool TRAIN>
__global__ __launch_bounds__(64) void fwd_state_kernel(
    const bf16* __restrict__ W, const bf16* __restrict__ UT, const bf16* __restrict__ KgT,
    const float* __restrict__ gc, const int32_t* __restrict__ chunks, const int32_t* __restrict__ doc_chunk,
    int H, const float* __restrict__ init_state, float* __restrict__ final_state, bf16* __restrict__ hT,
    bf16* __restrict__ hR, bf16* __restrict__ vnT, bf16* __restrict__ vnR) {
  const int h = blockIdx.x % H, slice = blockIdx.x / H, d = blockIdx.y;
  const int lane = threadIdx.x, r = lane & 15, q4 = lane >> 4;
  const int v0 = 16 * slice;

  f32x4 S[8];  // S[m][i] = state[k = 16m + 4q4 + i][v = v0 + r]
  if (init_state) {
    const float* s0 = init_state + ((size_t)d * H + h) * D * D;
#pragma unroll
    for (int m = 0; m < 8; ++m)
#pragma unroll
      for (int i = 0; i < 4; ++i) S[m][i] = s0[(16 * m + 4 * q4 + i) * D + v0 + r];
  } else {
#pragma unroll
    for (int m = 0; m < 8; ++m) S[m] = zero4();
  }

  const int c_end = doc_chunk[d + 1];
  for (int c = doc_chunk[d]; c < c_end; ++c) {
    const ChunkInfo ci = chunk_info(chunks, c);
    const size_t cb = (size_t)c * H + h;
    // state entering the chunk
    bf16* ht = hT + cb * (D * D);
#pragma unroll
    for (int m = 0; m < 8; ++m) st4(ht + (v0 + r) * D + 16 * m + 4 * q4, S[m]);
    if (TRAIN) {
      bf16* hr = hR + cb * (D * D);
#pragma unroll
      for (int m = 0; m < 8; ++m)
#pragma unroll
        for (int i = 0; i < 4; ++i) hr[(16 * m + 4 * q4 + i) * D + v0 + r] = (bf16)S[m][i];
    }
    bf16x8 hb[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) hb[j] = neg8(pack_perm(S[2 * j], S[2 * j + 1]));

    // v_new = U - W S   (rows t, 16 value columns)
    const bf16* ut = UT + cb * (D * CH);
    f32x4 vn[4];
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) {
      vn[i4] = cvtf4(ld4(ut + (v0 + r) * CH + 16 * i4 + 4 * q4));
      const int t = 16 * i4 + r;
      const bf16* wrow = W + ((size_t)(ci.start + t) * H + h) * D;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bf16x8 a = (t < ci.len) ? ld8p(wrow + 32 * j + 4 * q4) : zero8();
        vn[i4] = mfma(a, hb[j], vn[i4]);
      }
    }
    bf16* vt = vnT + cb * (D * CH);
#pragma unroll
    for (int i4 = 0; i4 < 4; ++i4) st4(vt + (v0 + r) * CH + 16 * i4 + 4 * q4, vn[i4]);
    if (TRAIN) {
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t = 16 * i4 + 4 * q4 + i;
          if (t < ci.len) vnR[((size_t)(ci.start + t) * H + h) * D + v0 + r] = (bf16)vn[i4][i];
        }
    }

    // S <- exp(G_last) S + (K exp(G_last - G))^T v_new
    const float gC = __expf(gc[(size_t)(ci.start + ci.len - 1) * H + h]);
    bf16x8 vb[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) vb[j] = pack_perm(vn[2 * j], vn[2 * j + 1]);
    const bf16* kg = KgT + cb * (D * CH);
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      S[m] *= gC;
#pragma unroll
      for (int j = 0; j < 2; ++j) S[m] = mfma(ld8p(kg + (16 * m + r) * CH + 32 * j + 4 * q4), vb[j], S[m]);
    }
  }
  if (final_state) {
    float* sf = final_state + ((size_t)d * H + h) * D * D;
#pragma unroll
    for (int m = 0; m < 8; ++m)
#pragma unroll
      for (int i = 0; i < 4; ++i) sf[(16 * m + 4 * q4 + i) * D + v0 + r] = S[m][i];
  }
}

// ---------------------------------------------------------------------------
// fwd_out: O^T (v rows, t columns) per chunk and head
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void fwd_out_kernel(
    const bf16* __restrict__ qn, const bf16* __restrict__ kn, const float* __restrict__ gc,
    const bf16* __restrict__ hT, const bf16* __restrict__ vnT, const int32_t* __restrict__ chunks, int H,
    float scale, bf16* __restrict__ o) {
  const int c = blockIdx.x, h = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r = lane & 15, q4 = lane >> 4;
  const ChunkInfo ci = chunk_info(chunks, c);
  const size_t cb = (size_t)c * H + h;

  __shared__ __attribute__((aligned(16))) bf16 Qs[64 * LDK];
  __shared__ __attribute__((aligned(16))) bf16 Ks[64 * LDK];
  __shared__ __attribute__((aligned(16))) bf16 Ps[64 * LDT];  // P[t][s], causal, gated
  __shared__ float Gs[64];

  {
    const int t = tid >> 2, p = tid & 3;
    const bool in = t < ci.len;
    const size_t row = ((size_t)(ci.start + t) * H + h) * D;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int col = 32 * j + 8 * p;
      st8(Qs + t * LDK + col, in ? ld8(qn + row + col) : zero8());
      st8(Ks + t * LDK + col, in ? ld8(kn + row + col) : zero8());
    }
    if (p == 0) Gs[t] = gc[(size_t)(ci.start + (in ? t : ci.len - 1)) * H + h];
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
  const bf16* ht = hT + cb * (D * D);
  const bf16* vt = vnT + cb * (D * CH);
  f32x4 acc[2][4];
#pragma unroll
  for (int mm = 0; mm < 2; ++mm)
#pragma unroll
    for (int n = 0; n < 4; ++n) acc[mm][n] = zero4();
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    bf16x8 bq[4];
#pragma unroll
    for (int n = 0; n < 4; ++n) bq[n] = ld8(Qs + (16 * n + r) * LDK + 32 * kb + 8 * q4);
#pragma unroll
    for (int mm = 0; mm < 2; ++mm) {
      const bf16x8 a = ld8(ht + (16 * (2 * wave + mm) + r) * D + 32 * kb + 8 * q4);
#pragma unroll
      for (int n = 0; n < 4; ++n) acc[mm][n] = mfma(a, bq[n], acc[mm][n]);
    }
  }
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    const float gam = __expf(Gs[16 * n + r]);
#pragma unroll
    for (int mm = 0; mm < 2; ++mm) acc[mm][n] *= gam;
  }
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    bf16x8 a[2];
#pragma unroll
    for (int mm = 0; mm < 2; ++mm) a[mm] = ld8(vt + (16 * (2 * wave + mm) + r) * CH + 32 * kb + 8 * q4);
#pragma unroll
    for (int n = 0; n < 4; ++n) {
      if (n < 2 * kb) continue;  // t-tile n holds no s in this block (s > t)
      const bf16x8 b = ld8(Ps + (16 * n + r) * LDT + 32 * kb + 8 * q4);
#pragma unroll
      for (int mm = 0; mm < 2; ++mm) acc[mm][n] = mfma(a[mm], b, acc[mm][n]);
    }
  }
#pragma unroll
  for (int n = 0; n < 4; ++n) {
    const int t = 16 * n + r;
    if (t >= ci.len) continue;
    bf16* orow = o + ((size_t)(ci.start + t) * H + h) * D;
#pragma unroll
    for (int mm = 0; mm < 2; ++mm) st4(orow + 16 * (2 * wave + mm) + 4 * q4, acc[mm][n] * scale);
  }
}

// ---------------------------------------------------------------------------
// host launchers
// ---------------------------------------------------------------------------
void launch_fwd(const FwdArgs& a, hipStream_t stream) {
  const dim3 grid_c(a.n_chunks, a.H);
  bf16* ws[F_COUNT];
  for (int i = 0; i < F_COUNT; ++i) ws[i] = reinterpret_cast<bf16*>(a.ws + a.off[i]);
  float* rq = reinterpret_cast<float*>(ws[F_RQ]);
  float* rk = reinterpret_cast<float*>(ws[F_RK]);
  float* gcum = reinterpret_cast<float*>(ws[F_GC]);
  if (a.normalize)
    hipLaunchKernelGGL(fwd_prep_kernel<true>, grid_c, dim3(256), 0, stream, a.q, a.k, a.v, a.g, a.beta, a.chunks,
                       a.H, ws[F_QN], ws[F_KN], rq, rk, gcum, ws[F_TM], ws[F_W], ws[F_WT], ws[F_UT], ws[F_KGT]);
  else
    hipLaunchKernelGGL(fwd_prep_kernel<false>, grid_c, dim3(256), 0, stream, a.q, a.k, a.v, a.g, a.beta, a.chunks,
                       a.H, ws[F_QN], ws[F_KN], rq, rk, gcum, ws[F_TM], ws[F_W], ws[F_WT], ws[F_UT], ws[F_KGT]);
  const dim3 grid_s(a.H * (D / 16), a.n_docs);
  if (a.training)
    hipLaunchKernelGGL(fwd_state_kernel<true>, grid_s, dim3(64), 0, stream, ws[F_W], ws[F_UT], ws[F_KGT], gcum,
                       a.chunks, a.doc_chunk, a.H, a.initial_state, a.final_state, ws[F_HT], ws[F_HR], ws[F_VNT],
                       ws[F_VN]);
  else
    hipLaunchKernelGGL(fwd_state_kernel<false>, grid_s, dim3(64), 0, stream, ws[F_W], ws[F_UT], ws[F_KGT], gcum,
                       a.chunks, a.doc_chunk, a.H, a.initial_state, a.final_state, ws[F_HT], ws[F_HR], ws[F_VNT],
                       ws[F_VN]);
  hipLaunchKernelGGL(fwd_out_kernel, grid_c, dim3(256), 0, stream, ws[F_QN], ws[F_KN], gcum, ws[F_HT], ws[F_VNT],
                     a.chunks, a.H, a.scale, a.o);
}

}  // namespace cqgdn
