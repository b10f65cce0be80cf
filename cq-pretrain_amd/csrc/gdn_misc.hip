// Memory-bound GDN kernels: the recurrent decode step, standalone l2norm
// forward/backward and the chunk-local (reverse) cumsum.
#include "gdn_common.hpp"
#include "gdn_kernels.hpp"

namespace cqgdn {

// ---------------------------------------------------------------------------
// recurrent: E events applied in order to each of N independent sequences.
// state is value-first [N][H][V][K] fp32 and is updated in place
// (ops/gated_delta_net.py:314-352, math of models/decoding.py:71-77):
//   S <- exp(g) S ;  r = (v - S k) * beta ;  S <- S + r k^T ;  o = scale * S q
// Two workgroups per (sequence, head), 64 state rows each, read once and
// written once per call whatever E is: the step is HBM-bound at 2 * 64 KB per
// (sequence, head).  A wave owns 16 rows; lane l holds columns 4 (l % 32) .. + 3
// of rows 2 jj + l / 32, so each load or store instruction of a wave covers
// 1 KB of contiguous state (two whole rows), and the row dot products are
// reduced over the 32 lanes of a row.  The state is streamed with
// non-temporal accesses: it is not reused before the next call.
// X: the element type of q, k, v and out (bf16, or fp16 read and written as
// such); every product and sum is in fp32 either way.
// ---------------------------------------------------------------------------
template <class X, bool BETA_BF16>
__global__ __launch_bounds__(256) void recurrent_kernel(const X* __restrict__ q, const X* __restrict__ k,
                                                        const X* __restrict__ v, const float* __restrict__ g,
                                                        const void* __restrict__ beta, float* __restrict__ state,
                                                        X* __restrict__ out, int E, int H, float scale) {
  const int blk = blockIdx.x;              // (n, h, half)
  const int half = blk & 1, nh = blk >> 1;  // nh = n * H + h
  const int n = nh / H, h = nh % H;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c4 = lane & 31;                                    // columns 4 c4 .. 4 c4 + 3
  const int rbase = 64 * half + 16 * wave + (lane >> 5);       // rows rbase + 2 jj
  float* sblk = state + (size_t)nh * D * D;
  f32x4 s[8];
#pragma unroll
  for (int jj = 0; jj < 8; ++jj)
    s[jj] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(sblk + (rbase + 2 * jj) * D + 4 * c4));
  for (int e = 0; e < E; ++e) {
    const size_t ev = ((size_t)n * E + e) * H + h;
    const float ge = __expf(g[ev]);
    const float be =
        BETA_BF16 ? (float)reinterpret_cast<const bf16*>(beta)[ev] : reinterpret_cast<const float*>(beta)[ev];
    const f32x4 kk = cvtf4(ld4(k + ev * D + 4 * c4));
    const f32x4 qq = cvtf4(ld4(q + ev * D + 4 * c4));
    float vv[8], o[8];
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) vv[jj] = (float)v[ev * D + rbase + 2 * jj];
    // four rows at a time: their row sums run level by level (no wait states between DPP
    // levels) and the cross-row step is a VALU swap, not an LDS-pipeline permute
#pragma unroll
    for (int j0 = 0; j0 < 8; j0 += 4) {
      float dot[4], od[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f32x4& sj = s[j0 + i];
        sj *= ge;
        dot[i] = sj[0] * kk[0] + sj[1] * kk[1] + sj[2] * kk[2] + sj[3] * kk[3];
      }
      sum16x4(dot);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f32x4& sj = s[j0 + i];
        sj += kk * ((vv[j0 + i] - sum_xor16(dot[i])) * be);
        od[i] = sj[0] * qq[0] + sj[1] * qq[1] + sj[2] * qq[2] + sj[3] * qq[3];
      }
      sum16x4(od);
#pragma unroll
      for (int i = 0; i < 4; ++i) o[j0 + i] = sum_xor16(od[i]);
    }
    if (c4 == 0) {
#pragma unroll
      for (int jj = 0; jj < 8; ++jj) out[ev * D + rbase + 2 * jj] = (X)(o[jj] * scale);
    }
  }
#pragma unroll
  for (int jj = 0; jj < 8; ++jj)
    __builtin_nontemporal_store(s[jj], reinterpret_cast<f32x4*>(sblk + (rbase + 2 * jj) * D + 4 * c4));
}

void launch_recurrent(const void* q, const void* k, const void* v, const float* g, const void* beta,
                      bool beta_bf16, bool fp16, float* state, void* out, int N, int E, int H, float scale,
                      hipStream_t stream) {
  const dim3 grid(2 * N * H);
  TimedLaunch tl(K_RECURRENT, stream);
  auto run = [&](auto x) {
    typedef decltype(x) X;
    const X* qx = static_cast<const X*>(q);
    const X* kx = static_cast<const X*>(k);
    const X* vx = static_cast<const X*>(v);
    X* ox = static_cast<X*>(out);
    if (beta_bf16)
      hipLaunchKernelGGL((recurrent_kernel<X, true>), grid, dim3(256), 0, stream, qx, kx, vx, g, beta, state, ox, E,
                         H, scale);
    else
      hipLaunchKernelGGL((recurrent_kernel<X, false>), grid, dim3(256), 0, stream, qx, kx, vx, g, beta, state, ox, E,
                         H, scale);
  };
  if (fp16)
    run(f16{});
  else
    run(bf16{});
}

// ---------------------------------------------------------------------------
// l2norm over rows of 128: y = x * rsqrt(sum x^2 + 1e-6); rstd saved for the
// backward dx = rstd * (dy - y (y . dy))  (K-a of the reference's op table,
// fla l2norm_fwd/bwd as called at ops/gated_delta_net.py:136-137,207-209).
// 16 threads per row, 8 elements each.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void l2norm_fwd_kernel(const bf16* __restrict__ x, bf16* __restrict__ y,
                                                         float* __restrict__ rstd, int64_t rows) {
  const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  const int c = threadIdx.x & 15;
  if (row >= rows) return;
  const f32x8 a = cvtf8(ld8(x + row * D + 8 * c));
  float ss = 0.f;
#pragma unroll
  for (int s = 0; s < 8; ++s) ss += a[s] * a[s];
  ss = sum16(ss);
  const float rs = rsqrtf(ss + 1e-6f);
  st8(y + row * D + 8 * c, cvt8(a * rs));
  if (c == 0 && rstd) rstd[row] = rs;
}

__global__ __launch_bounds__(256) void l2norm_bwd_kernel(const bf16* __restrict__ y, const float* __restrict__ rstd,
                                                         const bf16* __restrict__ dy, bf16* __restrict__ dx,
                                                         int64_t rows) {
  const int64_t row = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  const int c = threadIdx.x & 15;
  if (row >= rows) return;
  const f32x8 a = cvtf8(ld8(y + row * D + 8 * c));
  const f32x8 b = cvtf8(ld8(dy + row * D + 8 * c));
  float dot = 0.f;
#pragma unroll
  for (int s = 0; s < 8; ++s) dot += a[s] * b[s];
  dot = sum16(dot);
  st8(dx + row * D + 8 * c, cvt8((b - a * dot) * rstd[row]));
}

void launch_l2norm_fwd(const bf16* x, bf16* y, float* rstd, int64_t rows, hipStream_t stream) {
  const int64_t blocks = (rows + 15) / 16;
  hipLaunchKernelGGL(l2norm_fwd_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, x, y, rstd, rows);
}

void launch_l2norm_bwd(const bf16* y, const float* rstd, const bf16* dy, bf16* dx, int64_t rows,
                       hipStream_t stream) {
  const int64_t blocks = (rows + 15) / 16;
  hipLaunchKernelGGL(l2norm_bwd_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, y, rstd, dy, dx, rows);
}

// ---------------------------------------------------------------------------
// chunk-local cumsum of g [T][H] (forward or reverse) over the chunk table
// (K-b: chunk_local_cumsum / reverse_cumsum, ops/gated_delta_net.py:77-87,158-164)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void chunk_cumsum_kernel(const float* __restrict__ g, float* __restrict__ out,
                                                          const int32_t* __restrict__ chunks, int H, int reverse) {
  const int c = blockIdx.x, h = blockIdx.y, t = threadIdx.x;
  const ChunkInfo ci = chunk_info(chunks, c);
  const bool in = t < ci.len;
  float x = keep_if(in, g[(size_t)(ci.start + clamp_row(t, ci.len)) * H + h]);
  if (reverse) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float o = __shfl_down(x, off, 64);
      if (t + off < 64) x += o;
    }
  } else {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float o = __shfl_up(x, off, 64);
      if (t >= off) x += o;
    }
  }
  if (in) out[(size_t)(ci.start + t) * H + h] = x;
}

void launch_chunk_cumsum(const float* g, float* out, const int32_t* chunks, int n_chunks, int H, bool reverse,
                         hipStream_t stream) {
  hipLaunchKernelGGL(chunk_cumsum_kernel, dim3(n_chunks, H), dim3(64), 0, stream, g, out, chunks, H, (int)reverse);
}

__global__ __launch_bounds__(256) void copy_or_zero_kernel(float* __restrict__ dst, const float* __restrict__ src,
                                                           size_t n) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256)
    dst[i] = src ? src[i] : 0.f;
}

void launch_copy_or_zero(float* dst, const float* src, size_t n, hipStream_t stream) {
  const size_t blocks = (n + 255) / 256;
  hipLaunchKernelGGL(copy_or_zero_kernel, dim3((unsigned)(blocks < 4096 ? blocks : 4096)), dim3(256), 0, stream, dst,
                     src, n);
}

}  // namespace cqgdn
