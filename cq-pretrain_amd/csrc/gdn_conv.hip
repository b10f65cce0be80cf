// Packed depthwise causal conv1d, forward and backward (the GatedDelta layer's
// short conv over q/k/v channels, ops/gated_delta_net.py:252-289; the
// reference runs causal_conv1d_fn / causal_conv1d_bwd, models/backbone_qwen35.py
// keeps the CPU form F.conv1d(padding = K - 1) per document).
//
//   pre[t][c] = sum_{i<K} w[c][i] * x[t - (K-1) + i][c]   (rows of the same document only)
//   y = silu(pre) with the activation, else pre
//
// x, y, dy, dx: bf16 [T][C] (time-first, B = 1, packed documents); w: bf16
// [C][K], K <= 4.  A thread owns 8 consecutive channels (16-byte accesses, a
// wave covers 512 channels of one row: 1 KB per load or store) and walks a run
// of CONV_ROWS rows with a sliding window of the K - 1 previous rows; a window
// row from another document is zero.  Both passes are HBM-bound.
#include "gdn_common.hpp"
#include "gdn_kernels.hpp"

namespace cqgdn {

constexpr int CONV_ROWS = 32;     // rows per workgroup
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
struct DocCursor {
  const int32_t* bounds;
  int n, next, start;
  __device__ DocCursor(const int32_t* b, int n_docs, int u0) : bounds(b), n(n_docs) {
    int i = lower_bound(b, n_docs, u0 + 1) - 1;  // last bound <= u0
    i = max(i, 0);
    start = b[i];
    next = i + 1 <= n_docs ? i + 1 : n_docs;
  }
  __device__ __forceinline__ void advance_to(int u) {
    while (next <= n && bounds[next] <= u) start = bounds[next++];
  }
};

__device__ __forceinline__ float silu_f(float x) { return x / (1.f + __expf(-x)); }
__device__ __forceinline__ float dsilu_f(float x) {
  const float s = 1.f / (1.f + __expf(-x));
  return s * (1.f + x * (1.f - s));
}

template <int K>
__global__ __launch_bounds__(CONV_THREADS) void conv_fwd_kernel(const bf16* __restrict__ x, const bf16* __restrict__ w,
                                                               const int32_t* __restrict__ bounds, int n_docs,
                                                               int T, int C, int act, bf16* __restrict__ y) {
  const int c = (blockIdx.y * CONV_THREADS + threadIdx.x) * 8;
  if (c >= C) return;
  const int s = blockIdx.x * CONV_ROWS, e = min(s + CONV_ROWS, T);
  f32x8 wk[K];
  {
    const bf16* wc = w + (size_t)c * K;  // 8 channels x K taps, contiguous
#pragma unroll
    for (int ch = 0; ch < 8; ++ch)
#pragma unroll
      for (int i = 0; i < K; ++i) wk[i][ch] = (float)wc[ch * K + i];
  }
  f32x8 win[K];  // win[K-1-j] = x[u - j] (j = 0..K-1), rows of u's document
#pragma unroll
  for (int i = 0; i < K; ++i) win[i] = f32x8{};
  DocCursor doc(bounds, n_docs, max(s - (K - 1), 0));
  for (int u = max(s - (K - 1), 0); u < e; ++u) {
    const int prev_start = doc.start;
    doc.advance_to(u);
    if (doc.start != prev_start) {
#pragma unroll
      for (int i = 0; i < K; ++i) win[i] = f32x8{};
    }
#pragma unroll
    for (int i = 0; i < K - 1; ++i) win[i] = win[i + 1];
    win[K - 1] = cvtf8(ld8(x + (size_t)u * C + c));
    if (u >= s) {
      f32x8 acc = wk[0] * win[0];
#pragma unroll
      for (int i = 1; i < K; ++i) acc += wk[i] * win[i];
      if (act) {
#pragma unroll
        for (int ch = 0; ch < 8; ++ch) acc[ch] = silu_f(acc[ch]);
      }
      st8(y + (size_t)u * C + c, cvt8(acc));
    }
  }
}

// Backward over rows [s, e) of one workgroup: streams u from s - (K-1) to
// e + K - 2, recomputing pre[u] from the x window, dpre[u] = dy[u] * silu'(pre[u]);
// dw partials over u in [s, e); dx[t] for t = u - (K-1) once dpre[t .. t+K-1] is known:
//   dx[t] = sum_i w[i] * dpre[t + (K-1) - i]   (rows of t's document).
template <int K>
__global__ __launch_bounds__(CONV_THREADS) void conv_bwd_kernel(const bf16* __restrict__ x, const bf16* __restrict__ w,
                                                               const bf16* __restrict__ dy,
                                                               const int32_t* __restrict__ bounds, int n_docs,
                                                               int T, int C, int act, bf16* __restrict__ dx,
                                                               float* __restrict__ dw_part) {
  const int c = (blockIdx.y * CONV_THREADS + threadIdx.x) * 8;
  if (c >= C) return;
  const int s = blockIdx.x * CONV_ROWS, e = min(s + CONV_ROWS, T);
  f32x8 wk[K];
  {
    const bf16* wc = w + (size_t)c * K;
#pragma unroll
    for (int ch = 0; ch < 8; ++ch)
#pragma unroll
      for (int i = 0; i < K; ++i) wk[i][ch] = (float)wc[ch * K + i];
  }
  f32x8 xw[K], dp[K], dwa[K];
  int st[K];  // document start of each dpre window row
#pragma unroll
  for (int i = 0; i < K; ++i) {
    xw[i] = f32x8{};
    dp[i] = f32x8{};
    dwa[i] = f32x8{};
    st[i] = -1;
  }
  const int u0 = max(s - (K - 1), 0), u1 = min(e + K - 1, T);  // rows streamed: [u0, u1)
  DocCursor doc(bounds, n_docs, u0);
  for (int u = u0; u < u1 + K - 1; ++u) {
    f32x8 dpu = f32x8{};
    int stu = -2;  // no row (past the end)
    if (u < u1) {
      const int prev_start = doc.start;
      doc.advance_to(u);
      if (doc.start != prev_start) {
#pragma unroll
        for (int i = 0; i < K; ++i) xw[i] = f32x8{};
      }
#pragma unroll
      for (int i = 0; i < K - 1; ++i) xw[i] = xw[i + 1];
      xw[K - 1] = cvtf8(ld8(x + (size_t)u * C + c));
      stu = doc.start;
      if (u >= s) {
        dpu = cvtf8(ld8(dy + (size_t)u * C + c));
        if (act) {
          f32x8 pre = wk[0] * xw[0];
#pragma unroll
          for (int i = 1; i < K; ++i) pre += wk[i] * xw[i];
#pragma unroll
          for (int ch = 0; ch < 8; ++ch) dpu[ch] *= dsilu_f(pre[ch]);
        }
        if (u < e) {
#pragma unroll
          for (int i = 0; i < K; ++i) dwa[i] += dpu * xw[i];
        }
      }
    }
    // shift the dpre window: dp[K-1] = dpre[u], dp[0] = dpre[u - (K-1)]
#pragma unroll
    for (int i = 0; i < K - 1; ++i) {
      dp[i] = dp[i + 1];
      st[i] = st[i + 1];
    }
    dp[K - 1] = dpu;
    st[K - 1] = stu;
    const int t = u - (K - 1);
    if (t >= s && t < e) {
      // dpre[t + j] is dp[j]; tap i = K-1-j; same document: st[j] == st[0]
      f32x8 acc = wk[K - 1] * dp[0];
#pragma unroll
      for (int j = 1; j < K; ++j)
        if (st[j] == st[0]) acc += wk[K - 1 - j] * dp[j];
      st8(dx + (size_t)t * C + c, cvt8(acc));
    }
  }
  float* part = dw_part + ((size_t)blockIdx.x * C + c) * K;
#pragma unroll
  for (int ch = 0; ch < 8; ++ch)
#pragma unroll
    for (int i = 0; i < K; ++i) part[ch * K + i] = dwa[i][ch];
}

// dw[c][i] = sum over row tiles of the partials (fixed order: deterministic)
__global__ __launch_bounds__(256) void conv_dw_reduce_kernel(const float* __restrict__ part, int tiles, int n,
                                                            float* __restrict__ dw) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= n) return;
  float acc = 0.f;
  for (int b = 0; b < tiles; ++b) acc += part[(size_t)b * n + j];
  dw[j] = acc;
}

int conv_tiles(int64_t T) { return (int)((T + CONV_ROWS - 1) / CONV_ROWS); }

void launch_conv_fwd(const bf16* x, const bf16* w, const int32_t* bounds, int n_docs, int T, int C, int K, int act,
                     bf16* y, hipStream_t stream) {
  const dim3 grid(conv_tiles(T), (C / 8 + CONV_THREADS - 1) / CONV_THREADS);
  switch (K) {
    case 2: hipLaunchKernelGGL(conv_fwd_kernel<2>, grid, dim3(CONV_THREADS), 0, stream, x, w, bounds, n_docs, T, C, act, y); break;
    case 3: hipLaunchKernelGGL(conv_fwd_kernel<3>, grid, dim3(CONV_THREADS), 0, stream, x, w, bounds, n_docs, T, C, act, y); break;
    default: hipLaunchKernelGGL(conv_fwd_kernel<4>, grid, dim3(CONV_THREADS), 0, stream, x, w, bounds, n_docs, T, C, act, y); break;
  }
}

void launch_conv_bwd(const bf16* x, const bf16* w, const bf16* dy, const int32_t* bounds, int n_docs, int T, int C,
                     int K, int act, bf16* dx, float* dw, float* part, hipStream_t stream) {
  const int tiles = conv_tiles(T);
  const dim3 grid(tiles, (C / 8 + CONV_THREADS - 1) / CONV_THREADS);
  switch (K) {
    case 2: hipLaunchKernelGGL(conv_bwd_kernel<2>, grid, dim3(CONV_THREADS), 0, stream, x, w, dy, bounds, n_docs, T, C, act, dx, part); break;
    case 3: hipLaunchKernelGGL(conv_bwd_kernel<3>, grid, dim3(CONV_THREADS), 0, stream, x, w, dy, bounds, n_docs, T, C, act, dx, part); break;
    default: hipLaunchKernelGGL(conv_bwd_kernel<4>, grid, dim3(CONV_THREADS), 0, stream, x, w, dy, bounds, n_docs, T, C, act, dx, part); break;
  }
  const int n = C * K;
  hipLaunchKernelGGL(conv_dw_reduce_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, part, tiles, n, dw);
}

}  // namespace cqgdn
