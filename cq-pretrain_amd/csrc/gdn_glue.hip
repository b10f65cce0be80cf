// Kernels around the recurrence of one GatedDelta layer (models/backbone_qwen35.py:158-246):
// the gated RMSNorm fused with the output gather (ops/gated_delta_net.py:67-74 behind
// y.index_select(0, hidden_event), :242-246).
//
// Rows are [H][D = 128] bf16.  A (row, head) item is served by 16 lanes holding 8
// consecutive channels each (16-byte accesses; a wave covers 4 items = 1 KB), and
// its reductions are 16-lane butterflies, so every sum has a fixed order.
#include "gdn_common.hpp"
#include "gdn_kernels.hpp"

namespace cqgdn {

constexpr int GN_D = 128;
constexpr int GN_ITEMS = 16;  // (row, head) items per 256-thread workgroup

__device__ __forceinline__ float sigm(float x) { return __builtin_amdgcn_rcpf(1.f + __expf(-x)); }

__device__ __forceinline__ f32x8 ld_w8(const float* __restrict__ w, int l) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(w + l * 8);
  const f32x4 b = *reinterpret_cast<const f32x4*>(w + l * 8 + 4);
  return f32x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// out[r][h] = x * rsqrt(mean(x^2) + eps) * w * silu(z[r][h]),  x = y[index[r]][h] (0 if index[r] < 0)
__global__ __launch_bounds__(256) void gnorm_fwd_kernel(const bf16* __restrict__ y, const int32_t* __restrict__ index,
                                                       int64_t items, int H, const bf16* __restrict__ z,
                                                       int64_t z_stride, const float* __restrict__ w, float eps,
                                                       bf16* __restrict__ out, float* __restrict__ rstd) {
  const int64_t item = (int64_t)blockIdx.x * GN_ITEMS + (threadIdx.x >> 4);
  if (item >= items) return;  // whole 16-lane groups leave together
  const int l = threadIdx.x & 15;
  const int64_t r = item / H;
  const int h = (int)(item - r * H);
  const int64_t e = index ? (int64_t)index[r] : r;
  f32x8 v = f32x8{};
  if (e >= 0) v = cvtf8(ld8(y + (e * H + h) * GN_D + l * 8));
  const f32x8 zz = cvtf8(ld8(z + r * z_stride + h * GN_D + l * 8));
  const f32x8 wv = ld_w8(w, l);
  float ss = 0.f;
#pragma unroll
  for (int c = 0; c < 8; ++c) ss += v[c] * v[c];
  const float rs = __builtin_amdgcn_rsqf(sum16(ss) * (1.f / GN_D) + eps);
  f32x8 o;
#pragma unroll
  for (int c = 0; c < 8; ++c) o[c] = v[c] * rs * wv[c] * (zz[c] * sigm(zz[c]));
  st8(out + item * GN_D + l * 8, cvt8(o));
  if (l == 0) rstd[item] = rs;
}

// Backward of gnorm_fwd_kernel over items blk * 16 .. for blk = blockIdx.x, + gridDim.x, ...:
//   n = x * rstd, s = silu(z), dn = dout * w * s
//   dx = rstd * (dn - n * mean(dn * n))  -> dy[index[r]][h] (skipped for index < 0)
//   dz = dout * n * w * silu'(z)         -> dz[r][h] (row stride dz_stride)
//   dw partial of this workgroup = sum over its items of dout * n * s  -> wpart[blockIdx.x][128]
__global__ __launch_bounds__(256) void gnorm_bwd_kernel(const bf16* __restrict__ y, const int32_t* __restrict__ index,
                                                       int64_t items, int H, const bf16* __restrict__ z,
                                                       int64_t z_stride, const float* __restrict__ w,
                                                       const float* __restrict__ rstd, const bf16* __restrict__ dout,
                                                       bf16* __restrict__ dy, bf16* __restrict__ dz, int64_t dz_stride,
                                                       float* __restrict__ wpart) {
  __shared__ f32x8 red[GN_ITEMS][16];
  const int g = threadIdx.x >> 4, l = threadIdx.x & 15;
  const f32x8 wv = ld_w8(w, l);
  f32x8 dwa = f32x8{};
  for (int64_t blk = blockIdx.x; blk * GN_ITEMS < items; blk += gridDim.x) {
    const int64_t item = blk * GN_ITEMS + g;
    if (item < items) {  // uniform over the 16 lanes of the item
      const int64_t r = item / H;
      const int h = (int)(item - r * H);
      const int64_t e = index ? (int64_t)index[r] : r;
      f32x8 v = f32x8{};
      if (e >= 0) v = cvtf8(ld8(y + (e * H + h) * GN_D + l * 8));
      const f32x8 zz = cvtf8(ld8(z + r * z_stride + h * GN_D + l * 8));
      const f32x8 dd = cvtf8(ld8(dout + item * GN_D + l * 8));
      const float rs = rstd[item];
      f32x8 n, dn, dzv;
      float dot = 0.f;
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const float sg = sigm(zz[c]);
        const float s = zz[c] * sg;
        n[c] = v[c] * rs;
        dn[c] = dd[c] * wv[c] * s;
        dwa[c] += dd[c] * n[c] * s;
        dzv[c] = dd[c] * n[c] * wv[c] * (sg * (1.f + zz[c] * (1.f - sg)));
        dot += dn[c] * n[c];
      }
      dot = sum16(dot) * (1.f / GN_D);
      st8(dz + r * dz_stride + h * GN_D + l * 8, cvt8(dzv));
      if (e >= 0) {
        f32x8 dx;
#pragma unroll
        for (int c = 0; c < 8; ++c) dx[c] = rs * (dn[c] - n[c] * dot);
        st8(dy + (e * H + h) * GN_D + l * 8, cvt8(dx));
      }
    }
  }
  red[g][l] = dwa;
  __syncthreads();
  if (threadIdx.x < 16) {
    f32x8 acc = red[0][threadIdx.x];
    for (int q = 1; q < GN_ITEMS; ++q) acc += red[q][threadIdx.x];
    float* p = wpart + (size_t)blockIdx.x * GN_D + threadIdx.x * 8;
#pragma unroll
    for (int c = 0; c < 8; ++c) p[c] = acc[c];
  }
}

// rows[i] of x [.][row_elems] bf16 set to zero (row_elems % 8 == 0)
__global__ __launch_bounds__(256) void zero_rows_kernel(bf16* __restrict__ x, const int32_t* __restrict__ rows,
                                                       int64_t n, int row_elems) {
  const int per_row = row_elems / 8;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n * per_row) return;
  const int64_t k = i / per_row;
  const int j = (int)(i - k * per_row);
  st8(x + (int64_t)rows[k] * row_elems + j * 8, bf16x8{});
}

int gnorm_bwd_blocks(int64_t rows, int H) {
  const int64_t blocks = (rows * H + GN_ITEMS - 1) / GN_ITEMS;
  return (int)(blocks < 1024 ? blocks : 1024);
}

void launch_gnorm_fwd(const bf16* y, const int32_t* index, int64_t rows, int H, const bf16* z, int64_t z_stride,
                      const float* w, float eps, bf16* out, float* rstd, hipStream_t stream) {
  const int64_t items = rows * H;
  const dim3 grid((unsigned)((items + GN_ITEMS - 1) / GN_ITEMS));
  hipLaunchKernelGGL(gnorm_fwd_kernel, grid, dim3(256), 0, stream, y, index, items, H, z, z_stride, w, eps, out, rstd);
}

void launch_gnorm_bwd(const bf16* y, const int32_t* index, const int32_t* zero_rows, int64_t n_zero, int64_t rows,
                      int H, const bf16* z, int64_t z_stride, const float* w, const float* rstd, const bf16* dout,
                      bf16* dy, bf16* dz, int64_t dz_stride, float* dw, float* wpart, hipStream_t stream) {
  const int64_t items = rows * H;
  const int blocks = gnorm_bwd_blocks(rows, H);
  if (blocks > 0)
    hipLaunchKernelGGL(gnorm_bwd_kernel, dim3(blocks), dim3(256), 0, stream, y, index, items, H, z, z_stride, w,
                       rstd, dout, dy, dz, dz_stride, wpart);
  if (n_zero > 0) {
    const int64_t work = n_zero * (H * GN_D / 8);
    hipLaunchKernelGGL(zero_rows_kernel, dim3((unsigned)((work + 255) / 256)), dim3(256), 0, stream, dy, zero_rows,
                       n_zero, H * GN_D);
  }
  launch_colsum(wpart, blocks, GN_D, dw, stream);  // zeros when there are no rows
}

}  // namespace cqgdn
