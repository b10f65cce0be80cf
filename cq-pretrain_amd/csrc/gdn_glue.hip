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

// ---------------------------------------------------------------------------
// Event inputs of the recurrence (models/backbone_qwen35.py:166-194): the content
// conv output, the CQ query conv from the content history, the q/k/v gathers by
// event_q / event_write and the gate math, in one pass over the events; the
// backward walks the inverse maps, so every output row is written once and no
// atomics are used.  A workgroup has SV / 8 threads (SV = H * 128 value
// channels, 8 per thread); EvArgs documents the index arrays and the channel
// layout.  With fewer key heads than value heads the event rows repeat each
// key head for its G value heads, and the backward sums each group's q and k
// gradients (in fp32) into the key head's channels.

// key channel of value channel c: the same column of key head (c / 128) >> gshift
__device__ __forceinline__ int key_channel(int c, int gshift) { return (((c >> 7) >> gshift) << 7) | (c & 127); }

// first value channel of key channel c's group (the others follow 128 apart)
__device__ __forceinline__ int group_channel(int c, int gshift) { return (((c >> 7) << gshift) << 7) | (c & 127); }

__device__ __forceinline__ float softplus_f(float x) {  // torch's softplus (threshold 20)
  return x > 20.f ? x : log1pf(__expf(x));
}

// 8 channels x K taps of the conv weight [3S][K] as K fp32 vectors
template <int K>
__device__ __forceinline__ void ld_taps(const bf16* __restrict__ w, int c, f32x8 (&wk)[K]) {
  const bf16* wc = w + (size_t)c * K;
#pragma unroll
  for (int ch = 0; ch < 8; ++ch)
#pragma unroll
    for (int i = 0; i < K; ++i) wk[i][ch] = (float)wc[ch * K + i];
}

// pre-activation of query j's conv at channels c..c+7: its own raw row (tap K-1) and
// the history rows qhist[j][i] (content rows, read as raw rows order[.]; n_c = none)
template <int K>
__device__ __forceinline__ f32x8 query_pre(const EvArgs& a, int j, int c, const f32x8 (&wk)[K], f32x8 (&x)[K]) {
  x[K - 1] = cvtf8(ld8(a.raw + (int64_t)a.qsource[j] * a.raw_stride + c));
  f32x8 pre = wk[K - 1] * x[K - 1];
#pragma unroll
  for (int i = 0; i < K - 1; ++i) {
    const int hr = a.qhist[j * (K - 1) + i];
    x[i] = hr < a.n_c ? cvtf8(ld8(a.raw + (int64_t)a.order[hr] * a.raw_stride + c)) : f32x8{};
    pre += wk[i] * x[i];
  }
  return pre;
}

template <int K>
__global__ __launch_bounds__(512) void events_fwd_kernel(EvArgs a, const bf16* __restrict__ conv, bf16* __restrict__ q,
                                                        bf16* __restrict__ k, bf16* __restrict__ v,
                                                        float* __restrict__ g, float* __restrict__ beta) {
  const int e = blockIdx.x, SK = a.HK * GN_D, SV = a.H * GN_D, C = 2 * SK + SV, c = threadIdx.x * 8;
  const int ck = key_channel(c, a.gshift);
  const int sq = a.eq[e], sw = a.ew[e];
  bf16x8 q8;
  if (sq < a.n_c) {
    q8 = ld8(conv + (int64_t)sq * C + ck);
  } else {
    f32x8 wk[K], x[K];
    ld_taps<K>(a.w, ck, wk);
    f32x8 pre = query_pre<K>(a, sq - a.n_c, ck, wk, x);
#pragma unroll
    for (int ch = 0; ch < 8; ++ch) pre[ch] *= sigm(pre[ch]);
    q8 = cvt8(pre);
  }
  bf16x8 k8 = bf16x8{}, v8 = bf16x8{};
  if (sw < a.n_c) {
    k8 = ld8(conv + (int64_t)sw * C + SK + ck);
    v8 = ld8(conv + (int64_t)sw * C + 2 * SK + c);
  }
  st8(q + (int64_t)e * SV + c, q8);
  st8(k + (int64_t)e * SV + c, k8);
  st8(v + (int64_t)e * SV + c, v8);
  if (threadIdx.x < a.H) {
    const int h = threadIdx.x;
    float gv = 0.f, bv = 0.f;
    if (sw < a.n_c) {
      const int64_t row = a.order[sw];
      const float av = (float)a.ga[row * a.ga_stride + h] + a.dt_bias[h];
      gv = -__expf(a.A_log[h]) * softplus_f(av);
      bv = sigm((float)a.gb[row * a.gb_stride + h]);
    }
    g[(int64_t)e * a.H + h] = gv;
    beta[(int64_t)e * a.H + h] = bv;
  }
}

// content row cr: dconv[cr] = (sum of dq over the events reading q of cr, dk and dv of
// the event writing cr; q and k summed over each key head's value heads); gate
// gradients into the a/b columns of hidden row order[cr]; dA_log / dt_bias partials [cr][2H]
__global__ __launch_bounds__(512) void events_bwd_content_kernel(EvArgs a, EvGrads d, bf16* __restrict__ dconv,
                                                                float* __restrict__ gpart) {
  const int cr = blockIdx.x, SK = a.HK * GN_D, SV = a.H * GN_D, c = threadIdx.x * 8;
  const int we = a.winv[cr];
  bf16* out = dconv + (int64_t)cr * (2 * SK + SV);
  if (c < SK) {  // key channel c
    const int G = 1 << a.gshift, c0 = group_channel(c, a.gshift);
    f32x8 acc = f32x8{}, kacc = f32x8{};
    for (int p = a.qptr[cr]; p < a.qptr[cr + 1]; ++p) {
      const bf16* row = d.dq + (int64_t)a.qlist[p] * SV + c0;
      for (int g = 0; g < G; ++g) acc += cvtf8(ld8(row + g * GN_D));
    }
    if (we >= 0)
      for (int g = 0; g < G; ++g) kacc += cvtf8(ld8(d.dk + (int64_t)we * SV + c0 + g * GN_D));
    st8(out + c, cvt8(acc));
    st8(out + SK + c, cvt8(kacc));
  }
  st8(out + 2 * SK + c, we >= 0 ? ld8(d.dv + (int64_t)we * SV + c) : bf16x8{});
  if (threadIdx.x < a.H) {
    const int h = threadIdx.x;
    const int64_t row = a.order[cr];
    float da = 0.f, db = 0.f, dA = 0.f;
    if (we >= 0) {
      const float av = (float)a.ga[row * a.ga_stride + h] + a.dt_bias[h];
      const float ea = __expf(a.A_log[h]);
      const float dg = d.dg[(int64_t)we * a.H + h];
      da = -dg * ea * sigm(av);      // g = -exp(A_log) softplus(a + dt_bias)
      dA = -dg * ea * softplus_f(av);  // dg/dA_log = g
      const float sb = sigm((float)a.gb[row * a.gb_stride + h]);
      db = d.dbeta[(int64_t)we * a.H + h] * sb * (1.f - sb);
    }
    if (d.dcont) {
      d.dcgate[(int64_t)cr * 2 * a.H + h] = da;
      d.dcgate[(int64_t)cr * 2 * a.H + a.H + h] = db;
    } else {
      d.da[row * d.da_stride + h] = (bf16)da;
      d.db[row * d.db_stride + h] = (bf16)db;
    }
    gpart[(int64_t)cr * 2 * a.H + h] = dA;
    gpart[(int64_t)cr * 2 * a.H + a.H + h] = da;
  }
}

constexpr int EVQ_WAVES = 4;
// queries j = EVQ_WAVES blockIdx.x + wave, + EVQ_WAVES gridDim.x, ... for 512 key channels (blockIdx.y): dpre[j] =
// dq of the event reading j (summed over the key head's value heads) times silu'(pre); raw gradient of
// the query's own row (tap K-1; its k/v channels and gates get zeros); query-conv weight partials
// [blockIdx.x][SK][K].  The next query's dq rows and tap rows are requested before the current one computes.
template <int K>
__global__ __launch_bounds__(64 * EVQ_WAVES) void events_bwd_query_kernel(EvArgs a, EvGrads d,
                                                                        float* __restrict__ dpre,
                                                                        float* __restrict__ wpart) {
  // EVQ_WAVES waves per workgroup, each walking its own queries (the index
  // loads of a query are dependent, so queries in flight are what hides them);
  // the waves' weight partials are summed in LDS in a fixed order.
  const int SK = a.HK * GN_D, SV = a.H * GN_D, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = (blockIdx.y * 64 + lane) * 8, G = 1 << a.gshift, c0 = group_channel(c, a.gshift);
  f32x8 wk[K], dw[K];
  ld_taps<K>(a.w, c, wk);
#pragma unroll
  for (int i = 0; i < K; ++i) dw[i] = f32x8{};
  bf16x8 nq[EV_MAX_GROUP], nx[K];
  auto fetch = [&](int j) {
    const bf16* row = d.dq + (int64_t)a.qev[j] * SV + c0;
#pragma unroll
    for (int g = 0; g < EV_MAX_GROUP; ++g)
      if (g < G) nq[g] = ld8(row + g * GN_D);
    nx[K - 1] = ld8(a.raw + (int64_t)a.qsource[j] * a.raw_stride + c);
#pragma unroll
    for (int i = 0; i < K - 1; ++i) {
      const int hr = a.qhist[j * (K - 1) + i];
      nx[i] = hr < a.n_c ? ld8(a.raw + (int64_t)a.order[hr] * a.raw_stride + c) : bf16x8{};
    }
  };
  const int stride = EVQ_WAVES * (int)gridDim.x;
  int j = EVQ_WAVES * blockIdx.x + wave;
  if (j < a.n_q) fetch(j);
  for (; j < a.n_q; j += stride) {
    bf16x8 cq[EV_MAX_GROUP], cx[K];
#pragma unroll
    for (int g = 0; g < EV_MAX_GROUP; ++g) cq[g] = nq[g];
#pragma unroll
    for (int i = 0; i < K; ++i) cx[i] = nx[i];
    if (j + stride < a.n_q) fetch(j + stride);
    f32x8 x[K], pre = f32x8{};
#pragma unroll
    for (int i = 0; i < K; ++i) {
      x[i] = cvtf8(cx[i]);
      pre += wk[i] * x[i];
    }
    f32x8 dp = cvtf8(cq[0]);
#pragma unroll
    for (int g = 1; g < EV_MAX_GROUP; ++g)
      if (g < G) dp += cvtf8(cq[g]);
#pragma unroll
    for (int ch = 0; ch < 8; ++ch) {
      const float sg = sigm(pre[ch]);
      dp[ch] *= sg * (1.f + pre[ch] * (1.f - sg));
    }
    float* dpj = dpre + (int64_t)j * SK + c;
    *reinterpret_cast<f32x4*>(dpj) = f32x4{dp[0], dp[1], dp[2], dp[3]};
    *reinterpret_cast<f32x4*>(dpj + 4) = f32x4{dp[4], dp[5], dp[6], dp[7]};
#pragma unroll
    for (int i = 0; i < K; ++i) dw[i] += dp * x[i];
    const int64_t row = a.qsource[j];
    bf16* dr = d.draw + row * d.draw_stride;
    st8(dr + c, cvt8(dp * wk[K - 1]));
    st8(dr + SK + c, bf16x8{});
    for (int g = 0; g < G; ++g) st8(dr + 2 * SK + g * SK + c, bf16x8{});  // the SV = G SK value channels
    if (blockIdx.y == 0 && lane < a.H) {
      d.da[row * d.da_stride + lane] = (bf16)0.f;
      d.db[row * d.db_stride + lane] = (bf16)0.f;
    }
  }
  __shared__ f32x8 red[EVQ_WAVES - 1][K][64];  // waves 1 ..
  if (wave > 0) {
#pragma unroll
    for (int i = 0; i < K; ++i) red[wave - 1][i][lane] = dw[i];
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int w = 0; w < EVQ_WAVES - 1; ++w)
#pragma unroll
      for (int i = 0; i < K; ++i) dw[i] += red[w][i][lane];
    float* p = wpart + ((int64_t)blockIdx.x * SK + c) * K;
#pragma unroll
    for (int ch = 0; ch < 8; ++ch)
#pragma unroll
      for (int i = 0; i < K; ++i) p[ch * K + i] = dw[i][ch];
  }
}

// after the conv backward wrote the raw gradient of content row cr = hrows[blockIdx.x]:
// add the query convs' history taps, sum over (j, i) with qhist[j][i] == cr of dpre[j] w[., i]
// (key channels c: SK / 8 threads)
template <int K>
__global__ __launch_bounds__(512) void events_bwd_history_kernel(EvArgs a, EvGrads d, const float* __restrict__ dpre) {
  const int cr = a.hrows[blockIdx.x], SK = a.HK * GN_D, C = 2 * SK + a.H * GN_D, c = threadIdx.x * 8;
  f32x8 wk[K];
  ld_taps<K>(a.w, c, wk);
  f32x8 acc = f32x8{};
  for (int p = a.hptr[cr]; p < a.hptr[cr + 1]; ++p) {
    const int code = a.hlist[p], j = code / (K - 1), i = code - j * (K - 1);
    const float* dpj = dpre + (int64_t)j * SK + c;
    const f32x4 lo = *reinterpret_cast<const f32x4*>(dpj), hi = *reinterpret_cast<const f32x4*>(dpj + 4);
    f32x8 wi = wk[0];
#pragma unroll
    for (int t = 1; t < K - 1; ++t)
      if (i == t) wi = wk[t];
    acc += f32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]} * wi;
  }
  bf16* dr = d.dcont ? d.dcont + (int64_t)cr * C + c : d.draw + (int64_t)a.order[cr] * d.draw_stride + c;
  st8(dr, cvt8(cvtf8(ld8(dr)) + acc));
}

// Hidden row fold_rows[blockIdx.x], read by several content rows: its raw q|k|v
// gradient is the sum of theirs (ascending content row, fixed order), and its a
// and b gradients likewise -- the backward of the reference's
// raw.index_select(0, content_order) when content_order repeats a row.
__global__ __launch_bounds__(512) void events_bwd_fold_kernel(EvArgs a, EvGrads d) {
  const int row = d.fold_rows[blockIdx.x], C = (2 * a.HK + a.H) * GN_D;
  const int p0 = d.fold_ptr[blockIdx.x], p1 = d.fold_ptr[blockIdx.x + 1];
  bf16* dr = d.draw + (int64_t)row * d.draw_stride;
  for (int c = threadIdx.x * 8; c < C; c += blockDim.x * 8) {
    f32x8 acc = f32x8{};
    for (int p = p0; p < p1; ++p) acc += cvtf8(ld8(d.dcont + (int64_t)d.fold_list[p] * C + c));
    st8(dr + c, cvt8(acc));
  }
  if (threadIdx.x < 2 * a.H) {
    float acc = 0.f;
    for (int p = p0; p < p1; ++p) acc += d.dcgate[(int64_t)d.fold_list[p] * 2 * a.H + threadIdx.x];
    if (threadIdx.x < a.H)
      d.da[(int64_t)row * d.da_stride + threadIdx.x] = (bf16)acc;
    else
      d.db[(int64_t)row * d.db_stride + threadIdx.x - a.H] = (bf16)acc;
  }
}

__global__ __launch_bounds__(256) void add_f32_kernel(float* __restrict__ dst, const float* __restrict__ src, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) dst[i] += src[i];
}

int events_query_blocks(int n_q) { return n_q < 128 ? n_q : 128; }

void launch_events_fwd(const EvArgs& a, const bf16* conv, bf16* q, bf16* k, bf16* v, float* g, float* beta,
                       hipStream_t stream) {
  if (a.E == 0) return;
  const dim3 grid(a.E), block(a.H * 16);
  switch (a.K) {
    case 2: hipLaunchKernelGGL(events_fwd_kernel<2>, grid, block, 0, stream, a, conv, q, k, v, g, beta); break;
    case 3: hipLaunchKernelGGL(events_fwd_kernel<3>, grid, block, 0, stream, a, conv, q, k, v, g, beta); break;
    default: hipLaunchKernelGGL(events_fwd_kernel<4>, grid, block, 0, stream, a, conv, q, k, v, g, beta); break;
  }
}

void launch_events_bwd(const EvArgs& a, const EvGrads& d, const int32_t* content_bounds, int n_content_docs,
                       const EvWork& w, hipStream_t stream) {
  const int SK = a.HK * GN_D, C = 2 * SK + a.H * GN_D, H = a.H;
  const dim3 block(H * 16), kblock(a.HK * 16);
  if (a.n_c > 0) {
    hipLaunchKernelGGL(events_bwd_content_kernel, dim3(a.n_c), block, 0, stream, a, d, w.dconv, w.gpart);
  }
  const int qb = events_query_blocks(a.n_q);
  if (qb > 0) {
    const dim3 qgrid(qb, SK / 512);
    switch (a.K) {
      case 2: hipLaunchKernelGGL(events_bwd_query_kernel<2>, qgrid, dim3(64 * EVQ_WAVES), 0, stream, a, d, w.dpre, w.qpart); break;
      case 3: hipLaunchKernelGGL(events_bwd_query_kernel<3>, qgrid, dim3(64 * EVQ_WAVES), 0, stream, a, d, w.dpre, w.qpart); break;
      default: hipLaunchKernelGGL(events_bwd_query_kernel<4>, qgrid, dim3(64 * EVQ_WAVES), 0, stream, a, d, w.dpre, w.qpart); break;
    }
  }
  if (a.n_c > 0) {
    if (d.dcont)  // per-content-row gradients, folded into the hidden rows below
      launch_conv_bwd(a.raw, a.order, a.raw_stride, a.w, w.dconv, content_bounds, n_content_docs, a.n_c, C,
                      a.K, 1, d.dcont, nullptr, C, d.dw, w.cpart, stream);
    else
      launch_conv_bwd(a.raw, a.order, a.raw_stride, a.w, w.dconv, content_bounds, n_content_docs, a.n_c, C,
                      a.K, 1, d.draw, a.order, d.draw_stride, d.dw, w.cpart, stream);
  } else {
    launch_colsum(w.cpart, 0, C * a.K, d.dw, stream);  // zeros
  }
  if (a.n_hrows > 0) {
    switch (a.K) {
      case 2: hipLaunchKernelGGL(events_bwd_history_kernel<2>, dim3(a.n_hrows), kblock, 0, stream, a, d, w.dpre); break;
      case 3: hipLaunchKernelGGL(events_bwd_history_kernel<3>, dim3(a.n_hrows), kblock, 0, stream, a, d, w.dpre); break;
      default: hipLaunchKernelGGL(events_bwd_history_kernel<4>, dim3(a.n_hrows), kblock, 0, stream, a, d, w.dpre); break;
    }
  }
  if (d.dcont && d.n_fold > 0)
    hipLaunchKernelGGL(events_bwd_fold_kernel, dim3(d.n_fold), dim3(512), 0, stream, a, d);
  launch_colsum(w.gpart, a.n_c, 2 * H, d.dgate, stream);
  launch_colsum(w.qpart, qb, SK * a.K, w.qsum, stream);  // the query conv's taps: the q channels, first in dw
  hipLaunchKernelGGL(add_f32_kernel, dim3((SK * a.K + 255) / 256), dim3(256), 0, stream, d.dw, w.qsum, SK * a.K);
}


// ---------------------------------------------------------------------------
// One decode step of the layer for N independent sequences (models/decoding.py:16-78):
// row 0 of a sequence is the sampled content token C, row 1 the text-mask query Q.
//   C: pre = raw_C w[., K-1] + sum_j hist[j] w[., j] over the 3S channels, silu; the
//      history shifts by one row and takes raw_C
//   Q: the query conv of raw_Q's q channels over the updated history, silu
//   q (both rows) and k (C) l2-normalized; v = C's conv output; g, beta from C's a, b;
//   event 1 (Q) is read-only: k = v = 0, g = beta = 0, so its state update is the
//   identity and only its output is computed
//   recurrence (as recurrent_kernel): S <- exp(g) S; S <- S + k ((v - S k) beta)^T; o = scale S q
//   out = gated RMSNorm(o) with z from the row's projection (as gnorm_fwd_kernel)
// One launch, one workgroup of 8 waves per (sequence, value head h): head h's v
// channels and gates belong to its workgroup alone, and so do the q and k
// channels of its key head when key and value heads are equal; the waves own
// 16 state rows each (the layout of recurrent_kernel), so the head's whole output
// is in the workgroup for the norm.  q, k, v and o are rounded to bf16 where the
// separate kernels stored them, with the same 16- and 32-lane sums.  With G > 1
// value heads per key head, G workgroups read one key head's q and k history, so
// none of them shifts it: hist_shift_qk_kernel does, in a second launch.
template <int K>
__global__ __launch_bounds__(512) void decode_step_kernel(DecArgs a, float* __restrict__ state,
                                                          const float* __restrict__ norm_w, float eps, float scale,
                                                          bf16* __restrict__ out) {
  const int n = blockIdx.x / a.H, h = blockIdx.x % a.H, SK = a.HK * GN_D, SV = a.H * GN_D, C = 2 * SK + SV;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bf16* rc = a.proj + (int64_t)n * 2 * a.row_stride;  // the sampled token's row
  const bf16* rq = rc + a.row_stride;                       // the text-mask query's row
  __shared__ __attribute__((aligned(16))) float qs[2][GN_D], ks[GN_D], vs[GN_D], ys[2][GN_D];
  __shared__ float gb[2];
  if (tid < 48) {  // block p (q, k, v) of head h's channels: 16 lanes x 8 channels
    const int p = tid >> 4, l = tid & 15;
    const int c = (p == 2 ? 2 * SK + h * GN_D : p * SK + (h >> a.gshift) * GN_D) + l * 8;
    bf16* hist = a.hist + (int64_t)n * (K - 1) * C;
    f32x8 wk[K];
    ld_taps<K>(a.w, c, wk);
    const bf16x8 xc8 = ld8(rc + c);
    const f32x8 xc = cvtf8(xc8);
    bf16x8 h8[K - 1];
    f32x8 pre = wk[K - 1] * xc;
#pragma unroll
    for (int j = 0; j < K - 1; ++j) {
      h8[j] = ld8(hist + (int64_t)j * C + c);
      pre += wk[j] * cvtf8(h8[j]);
    }
#pragma unroll
    for (int ch = 0; ch < 8; ++ch) pre[ch] *= sigm(pre[ch]);
    f32x8 query = f32x8{};
    if (p == 0) {  // the query's conv sees the history after the token entered it
      query = wk[K - 1] * cvtf8(ld8(rq + c));
#pragma unroll
      for (int j = 0; j < K - 1; ++j) query += wk[j] * (j + 1 < K - 1 ? cvtf8(h8[j + 1]) : xc);
#pragma unroll
      for (int ch = 0; ch < 8; ++ch) query[ch] *= sigm(query[ch]);
    }
    if (p == 2 || a.gshift == 0) {
#pragma unroll
      for (int j = 0; j + 1 < K - 1; ++j) st8(hist + (int64_t)j * C + c, h8[j + 1]);
      st8(hist + (int64_t)(K - 2) * C + c, xc8);
    }
    float sp = 0.f, sqq = 0.f;
#pragma unroll
    for (int ch = 0; ch < 8; ++ch) {
      sp += pre[ch] * pre[ch];
      sqq += query[ch] * query[ch];
    }
    const float rp = __builtin_amdgcn_rsqf(sum16(sp) + 1e-6f), rqq = __builtin_amdgcn_rsqf(sum16(sqq) + 1e-6f);
    const f32x8 qc = cvtf8(cvt8(pre * rp)), qq = cvtf8(cvt8(query * rqq)), vr = cvtf8(cvt8(pre));
#pragma unroll
    for (int ch = 0; ch < 8; ++ch) {
      if (p == 0) {
        qs[0][l * 8 + ch] = qc[ch];
        qs[1][l * 8 + ch] = qq[ch];
      } else if (p == 1) {
        ks[l * 8 + ch] = qc[ch];
      } else {
        vs[l * 8 + ch] = vr[ch];
      }
    }
  } else if (tid == 64) {
    const float av = (float)rc[C + SV + h] + a.dt_bias[h];
    gb[0] = -__expf(a.A_log[h]) * softplus_f(av);
    gb[1] = sigm((float)rc[C + SV + a.H + h]);
  }
  __syncthreads();
  {
    const int c4 = lane & 31, rbase = 16 * wave + (lane >> 5);  // rows rbase + 2 jj
    float* sblk = state + ((size_t)n * a.H + h) * GN_D * GN_D;
    f32x4 st[8];
#pragma unroll
    for (int jj = 0; jj < 8; ++jj)
      st[jj] = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(sblk + (rbase + 2 * jj) * GN_D + 4 * c4));
    const float ge = __expf(gb[0]), be = gb[1];
    const f32x4 kk = *reinterpret_cast<const f32x4*>(&ks[4 * c4]);
    const f32x4 qc = *reinterpret_cast<const f32x4*>(&qs[0][4 * c4]);
    const f32x4 qq = *reinterpret_cast<const f32x4*>(&qs[1][4 * c4]);
    // four rows at a time: row sums level by level, cross-row steps on the VALU (as in
    // recurrent_kernel)
#pragma unroll
    for (int j0 = 0; j0 < 8; j0 += 4) {
      float dot[4], oc[4], oq[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f32x4& sj = st[j0 + i];
        sj *= ge;
        dot[i] = sj[0] * kk[0] + sj[1] * kk[1] + sj[2] * kk[2] + sj[3] * kk[3];
      }
      sum16x4(dot);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        f32x4& sj = st[j0 + i];
        sj += kk * ((vs[rbase + 2 * (j0 + i)] - sum_xor16(dot[i])) * be);
        oc[i] = sj[0] * qc[0] + sj[1] * qc[1] + sj[2] * qc[2] + sj[3] * qc[3];
        oq[i] = sj[0] * qq[0] + sj[1] * qq[1] + sj[2] * qq[2] + sj[3] * qq[3];
      }
      sum16x4(oc);
      sum16x4(oq);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float c = sum_xor16(oc[i]), qv = sum_xor16(oq[i]);
        if (c4 == 0) {
          ys[0][rbase + 2 * (j0 + i)] = (float)(bf16)(c * scale);
          ys[1][rbase + 2 * (j0 + i)] = (float)(bf16)(qv * scale);
        }
      }
    }
#pragma unroll
    for (int jj = 0; jj < 8; ++jj)
      __builtin_nontemporal_store(st[jj], reinterpret_cast<f32x4*>(sblk + (rbase + 2 * jj) * GN_D + 4 * c4));
  }
  __syncthreads();
  if (tid < 32) {  // gated RMSNorm of the token's (e = 0) and the query's (e = 1) output rows
    const int e = tid >> 4, l = tid & 15;
    const int64_t r = (int64_t)n * 2 + e;
    const f32x4 y0 = *reinterpret_cast<const f32x4*>(&ys[e][l * 8]), y1 = *reinterpret_cast<const f32x4*>(&ys[e][l * 8 + 4]);
    const f32x8 v = f32x8{y0[0], y0[1], y0[2], y0[3], y1[0], y1[1], y1[2], y1[3]};
    const f32x8 zz = cvtf8(ld8(a.proj + r * a.row_stride + C + h * GN_D + l * 8));
    const f32x8 wv = ld_w8(norm_w, l);
    float ss = 0.f;
#pragma unroll
    for (int c = 0; c < 8; ++c) ss += v[c] * v[c];
    const float rs = __builtin_amdgcn_rsqf(sum16(ss) * (1.f / GN_D) + eps);
    f32x8 o;
#pragma unroll
    for (int c = 0; c < 8; ++c) o[c] = v[c] * rs * wv[c] * (zz[c] * sigm(zz[c]));
    st8(out + (r * a.H + h) * GN_D + l * 8, cvt8(o));
  }
}

// The q and k history channels of sequence blockIdx.x shift by one row and take the
// sampled token's raw row (after decode_step_kernel has read them; 2 SK / 8 threads).
__global__ __launch_bounds__(1024) void hist_shift_qk_kernel(DecArgs a) {
  const int n = blockIdx.x, C = (2 * a.HK + a.H) * GN_D, c = threadIdx.x * 8;
  bf16* hist = a.hist + (int64_t)n * (a.K - 1) * C + c;
  for (int j = 0; j + 1 < a.K - 1; ++j) st8(hist + (int64_t)j * C, ld8(hist + (int64_t)(j + 1) * C));
  st8(hist + (int64_t)(a.K - 2) * C, ld8(a.proj + (int64_t)n * 2 * a.row_stride + c));
}

void launch_decode_step(const DecArgs& a, float* state, const float* norm_w, float eps, float scale, bf16* out,
                        hipStream_t stream) {
  if (a.N == 0) return;
  const dim3 grid(a.N * a.H), block(512);
  switch (a.K) {
    case 2: hipLaunchKernelGGL(decode_step_kernel<2>, grid, block, 0, stream, a, state, norm_w, eps, scale, out); break;
    case 3: hipLaunchKernelGGL(decode_step_kernel<3>, grid, block, 0, stream, a, state, norm_w, eps, scale, out); break;
    default: hipLaunchKernelGGL(decode_step_kernel<4>, grid, block, 0, stream, a, state, norm_w, eps, scale, out); break;
  }
  if (a.gshift > 0) hipLaunchKernelGGL(hist_shift_qk_kernel, dim3(a.N), dim3(a.HK * 32), 0, stream, a);
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
