// Packed depthwise causal conv1d, forward and backward (the GatedDelta layer's
// short conv over q/k/v channels, ops/gated_delta_net.py:252-289; the
// reference runs causal_conv1d_fn / causal_conv1d_bwd, models/backbone_qwen35.py
// keeps the CPU form F.conv1d(padding = K - 1) per document).
//
//   pre[t][c] = sum_{i<K} w[c][i] * x[t - (K-1) + i][c]   (rows of the same document only)
//   y = silu(pre) with the activation, else pre
//
// x, y, dy, dx: bf16 [T][C] (time-first, B = 1, packed documents); w: bf16
// [C][K], K <= 4.  Row u of x may be read through a row map (x row xrows[u],
// xs elements apart) and row t of dx written through its own map (dx row
// dxrows[t], dxs apart; null: row t):
// the layer's content gather updates = raw.index_select(0, content_order)
// (models/backbone_qwen35.py:167) and its backward, consumed in the loads and
// stores.  A thread owns 8 consecutive channels (16-byte accesses, a
// wave covers 512 channels of one row: 1 KB per load or store); a tap on a row
// of another document contributes nothing.  The forward requests every row of
// a CONV_ROWS tile (with the K - 1 row halo) before computing; the backward
// (CONV_BWD_CH channels per thread) streams longer strips with its loads one
// row group ahead, so that it writes few dw partials.  Both passes are
// HBM-bound.
#include "gdn_common.hpp"
#include "gdn_kernels.hpp"

#include <climits>

namespace cqgdn {

constexpr int CONV_ROWS = 16;     // rows per workgroup
constexpr int CONV_THREADS = 256; // 2048 channels per workgroup

// first index i with bounds[i] >= v (bounds ascending, n + 1 entries)
__device__ __forceinline__ int lower_bound(const int32_t* __restrict__ bounds, int n, int v) {
  int lo = 0, hi = n + 1;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (bounds[mid] < v) lo = mid + 1; else hi = mid;
  }
  return lo;
}

// Tracks the start of the document holding row u as u increases from u0.
// The next bound is kept in a register (nb), so a row that crosses no document
// boundary costs a compare, not a load and its wait.
struct DocCursor {
  const int32_t* bounds;
  int n, next, start, nb;  // nb = bounds[next], or INT_MAX past the last bound
  __device__ DocCursor(const int32_t* b, int n_docs, int u0) : bounds(b), n(n_docs) {
    int i = lower_bound(b, n_docs, u0 + 1) - 1;  // last bound <= u0
    i = max(i, 0);
    start = b[i];
    next = i + 1 <= n_docs ? i + 1 : n_docs;
    nb = next <= n ? b[next] : INT_MAX;
  }
  __device__ __forceinline__ void advance_to(int u) {
    while (nb <= u) {
      start = nb;
      ++next;
      nb = next <= n ? bounds[next] : INT_MAX;
    }
  }
};

// sigmoid through v_rcp_f32 (1 ulp) rather than an IEEE divide; exp(-x) = inf gives 0
__device__ __forceinline__ float sigmoid_f(float x) { return __builtin_amdgcn_rcpf(1.f + __expf(-x)); }
__device__ __forceinline__ float silu_f(float x) { return x * sigmoid_f(x); }
__device__ __forceinline__ float dsilu_f(float x) {
  const float s = sigmoid_f(x);
  return s * (1.f + x * (1.f - s));
}

template <int K>
__global__ __launch_bounds__(CONV_THREADS) void conv_fwd_kernel(const bf16* __restrict__ x, const int32_t* __restrict__ xrows,
                                                               int64_t xs, const bf16* __restrict__ w,
                                                               const int32_t* __restrict__ bounds, int n_docs,
                                                               int T, int C, int act, bf16* __restrict__ y) {
  const int c = (blockIdx.y * CONV_THREADS + threadIdx.x) * 8;
  if (c >= C) return;
  const int s = blockIdx.x * CONV_ROWS;
  const int u0 = s - (K - 1);
  // every row of the tile and its halo is requested before any is used
  bf16x8 xr[CONV_ROWS + K - 1];
#pragma unroll
  for (int i = 0; i < CONV_ROWS + K - 1; ++i) {
    const int u = min(max(u0 + i, 0), T - 1);  // rows outside [0, T) are never used
    xr[i] = ld8(x + (xrows ? (int64_t)xrows[u] : (int64_t)u) * xs + c);
  }
  f32x8 wk[K];
  {
    const bf16* wc = w + (size_t)c * K;  // 8 channels x K taps, contiguous
#pragma unroll
    for (int ch = 0; ch < 8; ++ch)
#pragma unroll
      for (int i = 0; i < K; ++i) wk[i][ch] = (float)wc[ch * K + i];
  }
  DocCursor doc(bounds, n_docs, max(s, 0));
#pragma unroll
  for (int r = 0; r < CONV_ROWS; ++r) {
    const int t = s + r;
    if (t >= T) break;
    doc.advance_to(t);
    f32x8 acc = f32x8{};
#pragma unroll
    for (int i = 0; i < K; ++i)  // tap i reads row t - (K-1) + i = xr[r + i]
      if (t - (K - 1) + i >= doc.start) acc += wk[i] * cvtf8(xr[r + i]);
    if (act) {
#pragma unroll
      for (int ch = 0; ch < 8; ++ch) acc[ch] = silu_f(acc[ch]);
    }
    st8(y + (size_t)t * C + c, cvt8(acc));
  }
}

// Backward: a one-wave workgroup streams a strip of rows [s, e) for
// 64 * CONV_BWD_CH channels, walking u = s - (K-1) .. e + K - 2 in groups of K rows whose x and
// dy rows are requested while the previous group computes.  Per row u:
//   pre[u] from the last K x rows, dpre[u] = dy[u] * silu'(pre[u]),
//   dw partials over u in [s, e),
//   dx[t] = sum_j w[K-1-j] * dpre[t + j] over rows t + j of t's document.
// The last K x rows (fp32) and dpre rows sit in rings indexed by the row's
// place in its group, so the windows advance without register moves.  A strip
// whose rows u0 .. uend-1 hold no document boundary (0 and T included) runs
// without any per-row document test (DOCS = false).  Each strip writes its dw
// partials [C][K]; colsum_kernel sums them.
constexpr int CONV_STRIPS = 128;  // row strips per 64 * CONV_BWD_CH channels
constexpr int CONV_BWD_CH = 4;    // channels per thread in the backward

template <int CH> struct ConvVec;
template <> struct ConvVec<8> { typedef bf16x8 b; typedef f32x8 f; };
template <> struct ConvVec<4> { typedef bf16x4 b; typedef f32x4 f; };

template <int K, int CH, bool DOCS>
__device__ __forceinline__ void conv_bwd_strip(const bf16* __restrict__ x, const int32_t* __restrict__ rows,
                                               int64_t xstr, const typename ConvVec<CH>::f (&wk)[K],
                                               const bf16* __restrict__ dy, const int32_t* __restrict__ bounds,
                                               int n_docs, int T, int C, int c, int s, int e, int act,
                                               bf16* __restrict__ dx, const int32_t* __restrict__ dxrows, int64_t dxs,
                                               typename ConvVec<CH>::f (&dwa)[K]) {
  typedef typename ConvVec<CH>::b bv;
  typedef typename ConvVec<CH>::f fv;
  const int u0 = s - (K - 1), uend = e + K - 1;
  bv nx[K], nd[K];  // the next group's rows (clamped into [0, T); rows outside are never used)
#pragma unroll
  for (int j = 0; j < K; ++j) {
    const int u = min(max(u0 + j, 0), T - 1);
    nx[j] = *reinterpret_cast<const bv*>(x + (rows ? (int64_t)rows[u] : (int64_t)u) * xstr + c);
    nd[j] = *reinterpret_cast<const bv*>(dy + (int64_t)u * C + c);
  }
  // ring slot j holds the row at place j of the current group (rows before u0 are never read)
  fv xs[K], dp[K];
  int st[K];  // document start of each dpre ring row (-1: no row)
#pragma unroll
  for (int i = 0; i < K; ++i) {
    dp[i] = fv{};
    st[i] = -1;
  }
  DocCursor doc(bounds, n_docs, s);
  for (int ub = u0; ub < uend; ub += K) {
    bv cx[K], cd[K];
#pragma unroll
    for (int j = 0; j < K; ++j) {
      cx[j] = nx[j];
      cd[j] = nd[j];
    }
    if (ub + K < uend) {
#pragma unroll
      for (int j = 0; j < K; ++j) {
        const int u = min(max(ub + K + j, 0), T - 1);
        nx[j] = *reinterpret_cast<const bv*>(x + (rows ? (int64_t)rows[u] : (int64_t)u) * xstr + c);
        nd[j] = *reinterpret_cast<const bv*>(dy + (int64_t)u * C + c);
      }
    }
#pragma unroll
    for (int j = 0; j < K; ++j) {
      const int u = ub + j;
      // slot j still holds row u - K until here: the taps of the rows before u read it
      xs[j] = __builtin_convertvector(cx[j], fv);
      if (u >= uend) break;
      if (u < s) continue;
      fv dpu = fv{};
      int stu = 0;
      if (!DOCS || u < T) {
        if (DOCS) {
          doc.advance_to(u);
          stu = __builtin_amdgcn_readfirstlane(doc.start);
        }
        // tap i reads row u - (K-1) + i, ring slot (j + 1 + i) % K
        fv pre = wk[K - 1] * xs[j];
#pragma unroll
        for (int i = 0; i < K - 1; ++i)
          if (!DOCS || u - (K - 1) + i >= stu) pre += wk[i] * xs[(j + 1 + i) % K];
        dpu = __builtin_convertvector(cd[j], fv);
        if (act) {
#pragma unroll
          for (int ch = 0; ch < CH; ++ch) dpu[ch] *= dsilu_f(pre[ch]);
        }
        if (u < e) {
          dwa[K - 1] += dpu * xs[j];
#pragma unroll
          for (int i = 0; i < K - 1; ++i)
            if (!DOCS || u - (K - 1) + i >= stu) dwa[i] += dpu * xs[(j + 1 + i) % K];
        }
      } else {
        stu = -1;
      }
      dp[j] = dpu;
      if (DOCS) st[j] = stu;
      const int t = u - (K - 1);
      if (t >= s && t < e) {  // dpre[t + m] is ring slot (j + 1 + m) % K, tap K-1-m, same document only
        fv acc = wk[K - 1] * dp[(j + 1) % K];
#pragma unroll
        for (int m = 1; m < K; ++m)
          if (!DOCS || st[(j + 1 + m) % K] == st[(j + 1) % K]) acc += wk[K - 1 - m] * dp[(j + 1 + m) % K];
        *reinterpret_cast<bv*>(dx + (dxrows ? (int64_t)dxrows[t] : (int64_t)t) * dxs + c) =
            __builtin_convertvector(acc, bv);
      }
    }
  }
}

template <int K>
__global__ __launch_bounds__(64) void conv_bwd_kernel(const bf16* __restrict__ x, const int32_t* __restrict__ xrows,
                                                     int64_t xs, const bf16* __restrict__ w,
                                                     const bf16* __restrict__ dy, const int32_t* __restrict__ bounds,
                                                     int n_docs, int T, int C, int rows, int act,
                                                     bf16* __restrict__ dx, const int32_t* __restrict__ dxrows,
                                                     int64_t dxs, float* __restrict__ dw_part) {
  constexpr int CH = CONV_BWD_CH;
  typedef typename ConvVec<CH>::f fv;
  const int c = (blockIdx.y * 64 + threadIdx.x) * CH;
  if (c >= C) return;
  const int s = blockIdx.x * rows, e = min(s + rows, T);
  fv wk[K], dwa[K];
  {
    const bf16* wc = w + (size_t)c * K;
#pragma unroll
    for (int ch = 0; ch < CH; ++ch)
#pragma unroll
      for (int i = 0; i < K; ++i) wk[i][ch] = (float)wc[ch * K + i];
  }
#pragma unroll
  for (int i = 0; i < K; ++i) dwa[i] = fv{};
  // a boundary b with u0 < b < uend separates two rows of the walk (b = 0 and b = T included)
  const int u0 = s - (K - 1), uend = e + K - 1;
  const int i = lower_bound(bounds, n_docs, u0 + 1);
  const bool docs = __builtin_amdgcn_readfirstlane(i <= n_docs && bounds[i] < uend);
  if (docs)
    conv_bwd_strip<K, CH, true>(x, xrows, xs, wk, dy, bounds, n_docs, T, C, c, s, e, act, dx, dxrows, dxs, dwa);
  else
    conv_bwd_strip<K, CH, false>(x, xrows, xs, wk, dy, bounds, n_docs, T, C, c, s, e, act, dx, dxrows, dxs, dwa);
  float* part = dw_part + ((size_t)blockIdx.x * C + c) * K;
#pragma unroll
  for (int ch = 0; ch < CH; ++ch)
#pragma unroll
    for (int k = 0; k < K; ++k) part[ch * K + k] = dwa[k][ch];
}

// dw[j] = sum over strips of the partials [strips][n] (n % 4 == 0; the conv's dw
// and the other per-workgroup parameter-gradient partials): a lane owns 4
// consecutive j (16-byte loads), a workgroup 256 j; its 4 waves sum strips
// b = wave, wave + 4, ... with 8 loads in flight, and the four sums are added
// in wave order (fixed order: deterministic).
__global__ __launch_bounds__(256) void colsum_kernel(const float* __restrict__ part, int strips, int n,
                                                    float* __restrict__ dw) {
  __shared__ f32x4 red[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = (blockIdx.x * 64 + lane) * 4;
  f32x4 acc = f32x4{};
  if (j < n) {
    const f32x4* p = reinterpret_cast<const f32x4*>(part + j);
    const size_t stride = (size_t)n / 4;
    int b = wave;
    for (; b + 28 < strips; b += 32) {
      f32x4 v[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) v[q] = p[(size_t)(b + 4 * q) * stride];
#pragma unroll
      for (int q = 0; q < 8; ++q) acc += v[q];
    }
    for (; b < strips; b += 4) acc += p[(size_t)b * stride];
  }
  red[wave][lane] = acc;
  __syncthreads();
  if (wave == 0 && j < n) {
    const f32x4 r = ((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane];
#pragma unroll
    for (int q = 0; q < 4; ++q) dw[j + q] = r[q];
  }
}

int conv_strip_rows(int64_t T) { return (int)std::max<int64_t>(16, (T + CONV_STRIPS - 1) / CONV_STRIPS); }

int conv_strips(int64_t T) {
  const int64_t rows = conv_strip_rows(T);
  return (int)((T + rows - 1) / rows);
}

void launch_conv_fwd(const bf16* x, const int32_t* xrows, int64_t xs, const bf16* w, const int32_t* bounds,
                     int n_docs, int T, int C, int K, int act, bf16* y, hipStream_t stream) {
  const dim3 grid((T + CONV_ROWS - 1) / CONV_ROWS, (C / 8 + CONV_THREADS - 1) / CONV_THREADS);
  switch (K) {
    case 2: hipLaunchKernelGGL(conv_fwd_kernel<2>, grid, dim3(CONV_THREADS), 0, stream, x, xrows, xs, w, bounds, n_docs, T, C, act, y); break;
    case 3: hipLaunchKernelGGL(conv_fwd_kernel<3>, grid, dim3(CONV_THREADS), 0, stream, x, xrows, xs, w, bounds, n_docs, T, C, act, y); break;
    default: hipLaunchKernelGGL(conv_fwd_kernel<4>, grid, dim3(CONV_THREADS), 0, stream, x, xrows, xs, w, bounds, n_docs, T, C, act, y); break;
  }
}

void launch_conv_bwd(const bf16* x, const int32_t* xrows, int64_t xs, const bf16* w, const bf16* dy,
                     const int32_t* bounds, int n_docs, int T, int C, int K, int act, bf16* dx, const int32_t* dxrows,
                     int64_t dxs, float* dw, float* part, hipStream_t stream) {
  const int rows = conv_strip_rows(T), strips = conv_strips(T);
  const dim3 grid(strips, (C / CONV_BWD_CH + 63) / 64);
  switch (K) {
    case 2: hipLaunchKernelGGL(conv_bwd_kernel<2>, grid, dim3(64), 0, stream, x, xrows, xs, w, dy, bounds, n_docs, T, C, rows, act, dx, dxrows, dxs, part); break;
    case 3: hipLaunchKernelGGL(conv_bwd_kernel<3>, grid, dim3(64), 0, stream, x, xrows, xs, w, dy, bounds, n_docs, T, C, rows, act, dx, dxrows, dxs, part); break;
    default: hipLaunchKernelGGL(conv_bwd_kernel<4>, grid, dim3(64), 0, stream, x, xrows, xs, w, dy, bounds, n_docs, T, C, rows, act, dx, dxrows, dxs, part); break;
  }
  launch_colsum(part, strips, C * K, dw, stream);
}

// The same sums for n <= 256 columns (n % 4 == 0) and many parts: one workgroup of
// 1024 threads, n / 4 float4 columns x 1024 / (n / 4) part stripes; each thread sums
// parts stripe, stripe + stripes, ... (8 loads in flight), then the stripes are
// added in stripe order.
__global__ __launch_bounds__(1024) void colsum_narrow_kernel(const float* __restrict__ part, int parts, int n,
                                                            float* __restrict__ out) {
  __shared__ f32x4 red[1024];
  const int n4 = n / 4, stripes = 1024 / n4;
  const int c4 = threadIdx.x % n4, stripe = threadIdx.x / n4;
  f32x4 acc = f32x4{};
  if (stripe < stripes) {
    const f32x4* p = reinterpret_cast<const f32x4*>(part) + c4;
    int b = stripe;
    for (; b + 7 * stripes < parts; b += 8 * stripes) {
      f32x4 v[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) v[q] = p[(size_t)(b + q * stripes) * n4];
#pragma unroll
      for (int q = 0; q < 8; ++q) acc += v[q];
    }
    for (; b < parts; b += stripes) acc += p[(size_t)b * n4];
  }
  red[threadIdx.x] = acc;
  __syncthreads();
  if (threadIdx.x < n4) {
    f32x4 r = red[threadIdx.x];
    for (int q = 1; q < stripes; ++q) r += red[q * n4 + threadIdx.x];
#pragma unroll
    for (int k = 0; k < 4; ++k) out[threadIdx.x * 4 + k] = r[k];
  }
}

void launch_colsum(const float* part, int parts, int n, float* out, hipStream_t stream) {
  if (n <= 256 && parts > 64)
    hipLaunchKernelGGL(colsum_narrow_kernel, dim3(1), dim3(1024), 0, stream, part, parts, n, out);
  else
    hipLaunchKernelGGL(colsum_kernel, dim3((n / 4 + 63) / 64), dim3(256), 0, stream, part, parts, n, out);
}

}  // namespace cqgdn
