// Shared device helpers for the gfx950 gated delta-rule (GDN) kernels.
//
// Every contraction runs on v_mfma_f32_16x16x32_bf16 (wave64).  Operand and
// result layouts of that instruction, as used throughout:
//
//   lane = threadIdx.x % 64, r = lane % 16, q4 = lane / 16 (0..3)
//   A operand (16 x 32, M x K):  lane holds A[m0 + r][k-slots of group q4]      (8 bf16)
//   B operand (32 x 16, K x N):  lane holds B[k-slots of group q4][n0 + r]      (8 bf16)
//   C/D       (16 x 16, M x N):  lane holds D[m0 + 4*q4 + i][n0 + r], i = 0..3  (4 fp32)
//
// The hardware pairs slot s of A with slot s of B, so which logical k a slot
// carries is ours to choose as long as A and B agree.  Two slot maps are used:
//   natural  : slot s of group q4 = k0 + 8*q4 + s              (one 16-byte load)
//   permuted : slot s of group q4 = k0 + 4*q4 + (s&3) + 16*(s>>2)
// The permuted map is what two stacked C tiles (rows k0..k0+15, k0+16..k0+31)
// already hold per lane, so an MFMA result feeds a following contraction over
// its M index straight from registers; the other operand is then fetched with
// two 8-byte loads (k0+4*q4.. and k0+16+4*q4..).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cqgdn {

constexpr int D = 128;   // head dimension (d_k = d_v), the only one the reference accepts
constexpr int CH = 64;   // chunk length of the WY/UT form

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }

__device__ __forceinline__ f32x4 mfma(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

// fp32 MFMA 16x16x4: lane (r, q4) holds A[r][q4] and B[q4][r]; the result has
// the layout of the 16x16x32 forms (C[4 q4 + i][r])
__device__ __forceinline__ f32x4 mfma4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 zero8() {
  bf16x8 z;
#pragma unroll
  for (int i = 0; i < 8; ++i) z[i] = (bf16)0.f;
  return z;
}

__device__ __forceinline__ bf16x4 cvt4(f32x4 x) { return __builtin_convertvector(x, bf16x4); }
__device__ __forceinline__ f32x4 cvtf4(bf16x4 x) { return __builtin_convertvector(x, f32x4); }
__device__ __forceinline__ f32x8 cvtf8(bf16x8 x) { return __builtin_convertvector(x, f32x8); }
__device__ __forceinline__ bf16x8 cvt8(f32x8 x) { return __builtin_convertvector(x, bf16x8); }

// Two C tiles (rows m0..m0+15 and m0+16..m0+31 of one column) -> one operand
// in the permuted slot map.
__device__ __forceinline__ bf16x8 pack_perm(f32x4 lo, f32x4 hi) {
  f32x8 x = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return cvt8(x);
}

__device__ __forceinline__ bf16x8 cat(bf16x4 a, bf16x4 b) {
  return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
}

__device__ __forceinline__ bf16x8 neg8(bf16x8 x) {
  // flip the sign bits (exact)
  u32x4 u = __builtin_bit_cast(u32x4, x);
  u ^= 0x80008000u;
  return __builtin_bit_cast(bf16x8, u);
}

// Storage order that makes a permuted-map fragment one contiguous 16-byte
// load: within every 32-element block, logical index x = 4q + s' + 16h
// (q = 0..3, s' = 0..3, h = 0..1) is stored at 8q + 4h + s'.  Tensors that
// are only ever read as permuted-map operands (W, KgT, W^T, the scan copy of
// Kn) are written in this order, so their consumers use ld8 at 32j + 8*q4.
__host__ __device__ __forceinline__ int perm32(int x) {
  return (x & ~31) | (((x >> 2) & 3) << 3) | (((x >> 4) & 1) << 2) | (x & 3);
}

// ---- fragment loads -------------------------------------------------------
// natural map, k-contiguous storage: 8 consecutive elements at p (16-byte aligned)
__device__ __forceinline__ bf16x8 ld8(const bf16* p) { return *reinterpret_cast<const bf16x8*>(p); }
__device__ __forceinline__ bf16x4 ld4(const bf16* p) { return *reinterpret_cast<const bf16x4*>(p); }
// The same 16 bytes loaded with the non-temporal hint (global_load ... nt): for
// input rows a kernel reads once, so that they do not displace, in the caches
// down to the memory-side cache, the data the next kernel reads.
__device__ __forceinline__ bf16x8 ld8_nt(const bf16* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const bf16x8*>(p));
}
// 16 bytes stored with the non-temporal hint: for whole rows written while the
// caches hold data the same kernel has yet to read.
__device__ __forceinline__ void st8_nt(bf16* p, bf16x8 x) {
  __builtin_nontemporal_store(x, reinterpret_cast<bf16x8*>(p));
}
// permuted map, k-contiguous storage: p points at element k0 + 4*q4
__device__ __forceinline__ bf16x8 ld8p(const bf16* p) { return cat(ld4(p), ld4(p + 16)); }
// natural map, strided storage: element s at p[s * stride]
__device__ __forceinline__ bf16x8 ld8s(const bf16* p, int stride) {
  bf16x8 x;
#pragma unroll
  for (int s = 0; s < 8; ++s) x[s] = p[s * stride];
  return x;
}

__device__ __forceinline__ void st4(bf16* p, f32x4 x) { *reinterpret_cast<bf16x4*>(p) = cvt4(x); }
__device__ __forceinline__ void st8(bf16* p, bf16x8 x) { *reinterpret_cast<bf16x8*>(p) = x; }

// Transposed fragment from a row-major LDS tile (row stride ld elements):
// lane (q4, r) gets tile[k0 + 8 q4 + e][n0 + r], e = 0..7 -- the natural-map
// operand for a contraction over the tile's row index.  Built from two
// ds_read_b64_tr_b16: within each 16-lane group, lane a addresses the 4
// elements tile[k0 + 8 q4 + 4 h + (a >> 2)][n0 + 4 (a & 3) ..], and the
// instruction returns to lane j element e of the group's lane (j >> 2) + 4 e,
// column j & 3 (the gfx950 layout, checked on the device).  tile must be in
// LDS, ld and n0 multiples of 4.
typedef short i16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ bf16x8 ld8_tr(const bf16* tile, int ld, int k0, int n0) {
  typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
  const int lane = threadIdx.x & 63, r = lane & 15, q4 = lane >> 4;
  const bf16* p = tile + (k0 + 8 * q4 + (r >> 2)) * ld + n0 + 4 * (r & 3);
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p + 4 * ld));
  return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

// C-layout column from a row-major LDS tile: lane (q4, r) gets tile[row0 + 4 q4 + e][col0 + r],
// e = 0..3 -- the rows and column an MFMA result fragment holds -- in one ds_read_b64_tr_b16:
// lane a of each 16-lane group addresses the 4 elements tile[row0 + 4 q4 + (a >> 2)][col0 +
// 4 (a & 3) ..], and the instruction hands lane j element e of lane (j >> 2) + 4 e, column
// j & 3 (the layout ld8_tr relies on).  ld and col0 multiples of 4.
__device__ __forceinline__ bf16x4 ld4_c(const bf16* tile, int ld, int row0, int col0) {
  typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
  const int lane = threadIdx.x & 63, r = lane & 15, q4 = lane >> 4;
  const bf16* p = tile + (row0 + 4 * q4 + (r >> 2)) * ld + col0 + 4 * (r & 3);
  return __builtin_bit_cast(bf16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p)));
}

// ---- fp16 operands ----------------------------------------------------------
// The precise (inference) forward, and the forward and backward of fp16 inputs,
// keep their MFMA operands in fp16: 11 mantissa bits instead of bf16's 8, at the
// same MFMA rate (v_mfma_f32_16x16x32_f16).  The kernels are templates over the
// operand element type E (bf16 or f16); Vec<E> names its vector types and the
// helpers below are overloaded on them.
typedef _Float16 f16;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4 mfma(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ f16x8 ld8(const f16* p) { return *reinterpret_cast<const f16x8*>(p); }
__device__ __forceinline__ f16x4 ld4(const f16* p) { return *reinterpret_cast<const f16x4*>(p); }
__device__ __forceinline__ f32x4 cvtf4(f16x4 x) { return __builtin_convertvector(x, f32x4); }
__device__ __forceinline__ f32x8 cvtf8(f16x8 x) { return __builtin_convertvector(x, f32x8); }
__device__ __forceinline__ f16x8 cat(f16x4 a, f16x4 b) { return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7); }
__device__ __forceinline__ void st4(f16* p, f32x4 x) {
  *reinterpret_cast<f16x4*>(p) = __builtin_convertvector(x, f16x4);
}
__device__ __forceinline__ void st8(f16* p, f16x8 x) { *reinterpret_cast<f16x8*>(p) = x; }

template <class E>
struct Vec;
template <>
struct Vec<bf16> {
  typedef bf16x8 x8;
  typedef bf16x4 x4;
};
template <>
struct Vec<f16> {
  typedef f16x8 x8;
  typedef f16x4 x4;
};

template <class E>
__device__ __forceinline__ typename Vec<E>::x4 to4(f32x4 x) {
  return __builtin_convertvector(x, typename Vec<E>::x4);
}
template <class E>
__device__ __forceinline__ typename Vec<E>::x8 to8(f32x8 x) {
  return __builtin_convertvector(x, typename Vec<E>::x8);
}
template <class E>
__device__ __forceinline__ typename Vec<E>::x8 zero8v() {
  return to8<E>(f32x8{});
}
// Eight values of a q or k input row as a kernel operand: E of float(x) * r,
// with r = rsqrt(sum x^2 + eps) of the row (1 without the in-kernel l2norm,
// where the product is exact).  fwd_prep forms its operands this way, so every
// kernel that reads q or k rounds them identically.
template <class E>
__device__ __forceinline__ typename Vec<E>::x8 scaled8(bf16x8 x, float r) {
  return to8<E>(cvtf8(x) * r);
}
// two C tiles -> one permuted-map operand (as pack_perm, for either element type)
template <class E>
__device__ __forceinline__ typename Vec<E>::x8 pack_permv(f32x4 lo, f32x4 hi) {
  return to8<E>(f32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]});
}

// ld8_tr for either operand element type
template <class E>
__device__ __forceinline__ typename Vec<E>::x8 ld8_trv(const E* tile, int ld, int k0, int n0) {
  typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
  const int lane = threadIdx.x & 63, r = lane & 15, q4 = lane >> 4;
  const E* p = tile + (k0 + 8 * q4 + (r >> 2)) * ld + n0 + 4 * (r & 3);
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p + 4 * ld));
  return __builtin_bit_cast(typename Vec<E>::x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

// ld8_tr with the rows in perm32 order: lane (q4, r) gets
// tile[k0 + 4 q4 + e][n0 + r] for e = 0..3 and tile[k0 + 16 + 4 q4 + e - 4][n0 + r]
// for e = 4..7, the K order of a B (or A) operand built by pack_perm from
// accumulator fragments.
template <class E>
__device__ __forceinline__ typename Vec<E>::x8 ld8_trpv(const E* tile, int ld, int k0, int n0) {
  typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
  const int lane = threadIdx.x & 63, r = lane & 15, q4 = lane >> 4;
  const E* p = tile + (k0 + 4 * q4 + (r >> 2)) * ld + n0 + 4 * (r & 3);
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p + 16 * ld));
  return __builtin_bit_cast(typename Vec<E>::x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}
__device__ __forceinline__ bf16x8 ld8_trp(const bf16* tile, int ld, int k0, int n0) {
  return ld8_trpv<bf16>(tile, ld, k0, n0);
}

// The fp16 forms of the bf16 helpers above, so that a kernel templated on its operand
// type calls them by one name: transposed fragments, non-temporal rows, and the
// operand rows of q and k formed from fp16 inputs.
__device__ __forceinline__ f16x8 ld8_tr(const f16* tile, int ld, int k0, int n0) {
  return ld8_trv<f16>(tile, ld, k0, n0);
}
__device__ __forceinline__ f16x8 ld8_trp(const f16* tile, int ld, int k0, int n0) {
  return ld8_trpv<f16>(tile, ld, k0, n0);
}
__device__ __forceinline__ f16x8 ld8_nt(const f16* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const f16x8*>(p));
}
__device__ __forceinline__ void st8_nt(f16* p, f16x8 x) {
  __builtin_nontemporal_store(x, reinterpret_cast<f16x8*>(p));
}
template <class E>
__device__ __forceinline__ typename Vec<E>::x8 scaled8(f16x8 x, float r) {
  return to8<E>(cvtf8(x) * r);
}

// Transposed read of a 16-row LDS tile [v][k] (row stride ld): lane (q4, r)
// gets tile[8 (q4 & 1) + e][k0 + 16 (q4 >> 1) + r], e = 0..7, i.e. 8
// consecutive rows of one column, for 32 columns k0 .. k0 + 31 per call.  Each
// 16-lane group transposes independently, so the groups take different row
// and column bases (ld8_tr's layout with the groups re-based).
template <class E>
__device__ __forceinline__ typename Vec<E>::x8 ld8_tr16(const E* tile, int ld, int k0) {
  typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
  const int lane = threadIdx.x & 63, r = lane & 15, q4 = lane >> 4;
  const E* p = tile + (8 * (q4 & 1) + (r >> 2)) * ld + k0 + 16 * (q4 >> 1) + 4 * (r & 3);
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p + 4 * ld));
  return __builtin_bit_cast(typename Vec<E>::x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

// Column gather of an MFMA fragment from a row-major bf16 matrix M in global
// memory (row stride ld, even; col0 even): lane (q4, r) gets
// M[row0 + 8 q4 + e][col0 + r], e = 0..7, 8 rows of one column, i.e. the
// fragment ld8 would give of M^T.  Lanes r and r ^ 1 share each dword: for rows
// 2i and 2i + 1 the even lane loads columns (r, r + 1) of row 2i and the odd
// lane columns (r - 1, r) of row 2i + 1; the pair swaps the loaded dwords
// through DPP and each keeps its own column's halves (v_perm).  Every load
// instruction reads 8 runs of 32 bytes.
//
// It comes in two steps, col8_load and col8_combine: the exchange has to wait
// for the loads, so a caller with more loads to issue puts them between the two
// steps and pays one memory round trip for all of them.
struct Col8 {
  uint32_t x[4];
};
__device__ __forceinline__ Col8 col8_load(const bf16* M, int ld, int row0, int col0) {
  const int lane = threadIdx.x & 63, r = lane & 15, q4 = lane >> 4, odd = r & 1;
  const uint32_t* p = reinterpret_cast<const uint32_t*>(M + (size_t)(row0 + 8 * q4 + odd) * ld + col0 + r - odd);
  Col8 g;
#pragma unroll
  for (int i = 0; i < 4; ++i) g.x[i] = p[i * ld];  // rows 2i + odd, ld / 2 dwords per row pair
  return g;
}
// col8_load over rows [0, nrows) of M (row stride ld): rows past nrows read
// row nrows - 1 instead (in bounds, values unspecified: the caller zeroes them
// or multiplies them by zero).
__device__ __forceinline__ Col8 col8_load_rows(const bf16* M, int ld, int row0, int col0, int nrows) {
  const int lane = threadIdx.x & 63, r = lane & 15, q4 = lane >> 4, odd = r & 1;
  Col8 g;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = min(row0 + 8 * q4 + 2 * i + odd, nrows - 1);
    g.x[i] = *reinterpret_cast<const uint32_t*>(M + (size_t)row * ld + col0 + r - odd);
  }
  return g;
}
__device__ __forceinline__ bf16x8 col8_combine(const Col8& g) {
  const int odd = threadIdx.x & 1;
  // {S0 = partner, S1 = own}: even keeps own low halves, odd keeps own high halves
  const uint32_t sel = odd ? 0x03020706u : 0x05040100u;
  u32x4 out;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t y = (uint32_t)__builtin_amdgcn_mov_dpp((int)g.x[i], 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
    out[i] = __builtin_amdgcn_perm(y, g.x[i], sel);
  }
  return __builtin_bit_cast(bf16x8, out);
}
__device__ __forceinline__ bf16x8 gather8_col_rows(const bf16* M, int ld, int row0, int col0, int nrows) {
  return col8_combine(col8_load_rows(M, ld, row0, col0, nrows));
}
// The same gathers over an fp16 matrix (they move 16-bit values without looking at them)
__device__ __forceinline__ Col8 col8_load(const f16* M, int ld, int row0, int col0) {
  return col8_load(reinterpret_cast<const bf16*>(M), ld, row0, col0);
}
__device__ __forceinline__ Col8 col8_load_rows(const f16* M, int ld, int row0, int col0, int nrows) {
  return col8_load_rows(reinterpret_cast<const bf16*>(M), ld, row0, col0, nrows);
}
template <class E>
__device__ __forceinline__ typename Vec<E>::x8 col8_combine_v(const Col8& g) {
  return __builtin_bit_cast(typename Vec<E>::x8, col8_combine(g));
}

// ---- workgroup synchronization for loader/consumer kernels ----------------
// Barrier that orders LDS only: waits for this wave's LDS operations, then
// s_barrier.  __syncthreads() also waits for every outstanding vector-memory
// operation (including asynchronous global->LDS copies still in flight for
// later steps), which would serialize a prefetch pipeline.  The "memory"
// clobber keeps the compiler from moving memory accesses across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Wait until every vector-memory operation this wave issued has completed.
__device__ __forceinline__ void wait_vmem_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }  // vmcnt(0)

// Wait until at most N of this wave's vector-memory operations are in flight.
// On gfx9 loads and stores share one counter and retire in issue order, so
// this waits for everything issued before the last N operations.
template <int N>
__device__ __forceinline__ void wait_vmem_le() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt(0x0F70 | (N & 15) | ((N >> 4) << 14));
}

// vmcnt(parts * P + stores * S) for counts known only at run time (parts and
// stores in 0..2): the wait of a wave that has issued `parts` copy parts of P
// operations and `stores` store groups of S since the operations it waits for.
template <int P, int S>
__device__ __forceinline__ void wait_vmem_parts(int parts, int stores) {
  static_assert(2 * P + 2 * S < 64, "vmcnt is 6 bits");
  switch (parts * 3 + stores) {
    case 0: wait_vmem_le<0>(); break;
    case 1: wait_vmem_le<S>(); break;
    case 2: wait_vmem_le<2 * S>(); break;
    case 3: wait_vmem_le<P>(); break;
    case 4: wait_vmem_le<P + S>(); break;
    case 5: wait_vmem_le<P + 2 * S>(); break;
    case 6: wait_vmem_le<2 * P>(); break;
    case 7: wait_vmem_le<2 * P + S>(); break;
    default: wait_vmem_le<2 * P + 2 * S>(); break;
  }
}

// Hand-off counters in LDS between the waves of one workgroup, in place of
// s_barrier: a producer wave publishes a count once everything it covers is in
// LDS (its own LDS operations complete in order, and an asynchronous copy has
// landed once vmcnt says so); a consumer wave polls the count.  Every wait is
// bounded: after FLAG_SPIN_LIMIT polls it gives up and returns false, so a
// broken hand-off ends the kernel with wrong results instead of hanging it.
// The casts name the LDS address space: through a plain volatile pointer the
// accesses would become flat operations that wait for every vector memory
// operation in flight (a loader's own copies included).
constexpr int FLAG_SPIN_LIMIT = 1 << 20;
typedef __attribute__((address_space(3))) volatile int lds_vint;
typedef __attribute__((address_space(3))) volatile long long lds_vi64;
__device__ __forceinline__ int lds_flag_read(const int* f) {
  return __builtin_amdgcn_readfirstlane(*(lds_vint*)(f));
}
__device__ __forceinline__ void lds_flag_publish(int* f, int v) {
  asm volatile("" ::: "memory");
  *(lds_vint*)(f) = v;
  asm volatile("" ::: "memory");
}
// two adjacent counts in one LDS read
__device__ __forceinline__ int2 lds_flag_read2(const int* f) {
  const long long v = *(lds_vi64*)(f);
  return int2{(int)v, (int)(v >> 32)};
}
template <bool SLEEP>
__device__ __forceinline__ bool lds_flag_wait_ge(const int* f, int target) {
  for (int i = 0; i < FLAG_SPIN_LIMIT; ++i) {
    if (lds_flag_read(f) >= target) {
      asm volatile("" ::: "memory");
      return true;
    }
    if (SLEEP) __builtin_amdgcn_s_sleep(1);
  }
  return false;
}

// A scan consumer's wait for step target-1 from both of its loaders (counts
// flags[0], flags[1]); `seen` gets the smaller count read.  Bounded (see
// lds_flag_wait_ge): false if it gave up.
__device__ __forceinline__ bool scan_wait_ready(const int* flags, int target, int& seen) {
  for (int i = 0; i < FLAG_SPIN_LIMIT; ++i) {
    const int2 v = lds_flag_read2(flags);
    const int mn = min(__builtin_amdgcn_readfirstlane(v.x), __builtin_amdgcn_readfirstlane(v.y));
    if (mn >= target) {
      asm volatile("" ::: "memory");
      seen = mn;
      return true;
    }
  }
  return false;
}

typedef __attribute__((address_space(3))) void* lds_void_ptr;

// Asynchronous copy global -> LDS, 16 bytes per lane: lane l's 16 bytes land at
// lds + 16*l (lds must be wave-uniform and 16-byte aligned).
__device__ __forceinline__ void dma16(const void* src, void* lds) {
  __builtin_amdgcn_global_load_lds(src, (lds_void_ptr)lds, 16, 0, 0);
}

// ---- power-of-two range scales of the fp16 paths ---------------------------
// The scale of V (or dO) is 2^(target - e) for the e with max|x| in [2^(e-1), 2^e),
// and 1 when every value is zero or one is not finite.  A pass over x leaves 1024
// partial maxima in scale[1 .. 1024]; the first kernel that needs the scale forms it
// in each of its 256-thread workgroups, thread i contributing the largest of partials
// i, i + 256, i + 512, i + 768 (range_partial4), and one workgroup stores it in
// scale[0] for the kernels after it.  Every thread of the workgroup calls
// range_scale (it holds a barrier); red: 4 floats of LDS.
__device__ __forceinline__ float range_partial4(const float* part) {
  const int i = threadIdx.x;
  return fmaxf(fmaxf(part[i], part[i + 256]), fmaxf(part[i + 512], part[i + 768]));
}
__device__ __forceinline__ float range_scale(float m, int target, float* red) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  lds_barrier();  // orders LDS only: the caller's global loads stay in flight
  m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float sc = 1.f;
  if (m > 0.f && isfinite(m)) {
    int e;
    frexpf(m, &e);  // m < 2^e
    sc = ldexpf(1.f, min(max(target - e, -60), 60));
  }
  return sc;
}

// ---- wave reductions -------------------------------------------------------
// x of another lane of the same 16-lane row, by a DPP control (VALU only, no LDS)
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}

// sum over the 16 lanes that share q4 (the 16 columns of a C tile), as a pairwise
// tree of DPP moves: lane ^ 1 and lane ^ 2 (quad_perm), then lane ^ 15 (row_mirror)
// and lane ^ 7 (row_half_mirror).  Every level adds a + b on one lane and b + a on
// its partner, so all 16 lanes hold the same bits.
__device__ __forceinline__ float sum16(float x) {
  x += dpp_f<0xB1>(x);   // quad_perm [1, 0, 3, 2]
  x += dpp_f<0x4E>(x);   // quad_perm [2, 3, 0, 1]
  x += dpp_f<0x140>(x);  // row_mirror
  x += dpp_f<0x141>(x);  // row_half_mirror
  return x;
}

// sum over the four 16-lane rows (lanes r, r + 16, r + 32, r + 48: the 4 row groups of a
// C tile), with v_permlane16_swap and v_permlane32_swap (VALU; no LDS round trip).  With
// both operands holding x, a swap leaves rows {x0, x0, x2, x2} in the first and {x1, x1,
// x3, x3} in the second (permlane16; permlane32 likewise with the two halves), so adding
// them gives every lane the same bits: (x0 + x1) + (x2 + x3), as x + xor16(x), then + xor32.
// Written as assembly with two tied operands because this compiler's builtin drops the
// second result when both inputs are the same value; the s_nops give the swaps their
// VALU hazard distance on both sides.
// The leading s_nop 1 gives the swap's operands, which a VALU copy has just written, the
// two wait states a VALU write needs before a permlane reads it (the compiler cannot place
// hazard waits inside inline assembly); the swap's results may be read at once (this
// compiler's own schedule for the builtin reads them in the next instruction).
__device__ __forceinline__ float sum_rows4(float x) {
  float a = x, b = x;
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  x = a + b;
  float c = x, d = x;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(c), "+v"(d));
  return c + d;
}

// x + x from lane ^ 16 (the sum over 16-lane rows 2i and 2i + 1), bit for bit the same as
// x + __shfl_xor(x, 16) (the addition commutes), on the VALU: v_permlane16_swap with both
// operands holding x leaves row 2i's value in one and row 2i + 1's in the other, instead of
// a ds_bpermute round trip through the LDS pipeline
__device__ __forceinline__ float sum_xor16(float x) {
  float a = x, b = x;
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  return a + b;
}

// c + sum of a[e] b[e] over 8 bf16 pairs, as four v_dot2_f32_bf16 (products and sums in fp32)
__device__ __forceinline__ float dot8(bf16x8 a, bf16x8 b, float c) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
#pragma unroll
  for (int e = 0; e < 8; e += 2)
    c = __builtin_amdgcn_fdot2_f32_bf16(bf16x2{a[e], a[e + 1]}, bf16x2{b[e], b[e + 1]}, c, false);
  return c;
}
// the same over 8 fp16 pairs (v_dot2_f32_f16)
__device__ __forceinline__ float dot8(f16x8 a, f16x8 b, float c) {
  typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
#pragma unroll
  for (int e = 0; e < 8; e += 2) c = __builtin_amdgcn_fdot2(f16x2{a[e], a[e + 1]}, f16x2{b[e], b[e + 1]}, c, false);
  return c;
}

// sum16 of four independent values, level by level (each value gets the same operations in
// the same order as sum16): a DPP move then reads a register written three instructions
// earlier, so the levels need no wait states between them (one value at a time, every level
// waits two cycles for the previous one)
__device__ __forceinline__ void sum16x4(float (&x)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) x[i] += dpp_f<0xB1>(x[i]);
#pragma unroll
  for (int i = 0; i < 4; ++i) x[i] += dpp_f<0x4E>(x[i]);
#pragma unroll
  for (int i = 0; i < 4; ++i) x[i] += dpp_f<0x140>(x[i]);
#pragma unroll
  for (int i = 0; i < 4; ++i) x[i] += dpp_f<0x141>(x[i]);
}

// sum over the 4 lanes of a quad (lanes 4a .. 4a + 3), the first two levels of sum16
__device__ __forceinline__ float sum4(float x) {
  x += dpp_f<0xB1>(x);
  x += dpp_f<0x4E>(x);
  return x;
}

// The l2 scale rsqrt(sum x^2 + 1e-6) of an event row of q or k, whose 128 values
// four adjacent threads hold as 8-value pieces (columns 32 j + 8 p of row t for
// thread 4 t + p).  Every kernel that reads q or k rows in this layout forms the
// scale itself, with the same sums in the same order, so all of them apply the
// same bits and no kernel stores it.
template <class X8>
__device__ __forceinline__ float row_rnorm(const X8 (&x)[4]) {
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const f32x8 y = cvtf8(x[j]);
#pragma unroll
    for (int s = 0; s < 8; ++s) ss += y[s] * y[s];
  }
  return rsqrtf(sum4(ss) + 1e-6f);
}

// Rows past a tail chunk's length re-read the chunk's last row (always in bounds)
// and are zeroed after the load.  A load issued under a condition is waited for
// on its own (the compiler branches around it); unconditional loads of a phase
// are all issued before the first wait.
__device__ __forceinline__ int clamp_row(int t, int len) { return t < len ? t : len - 1; }
template <class V>
__device__ __forceinline__ V keep_if(bool in, V x) {
  return in ? x : V{};
}

// ---- chunk-row stores through a buffer resource ----------------------------
// A raw buffer resource over the rows of one chunk in an [events][H][128] bf16
// tensor: based at head h of the chunk's first event, it ends after the last
// valid row, so the hardware's range check drops stores to rows past the chunk's
// length (no per-lane branch).  A store's address is a per-lane VGPR offset plus a
// wave-uniform SGPR offset (the row), instead of a 64-bit address per lane.
// 0x00020000 is the resource's fourth dword for a raw buffer on gfx9-family parts.
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
template <class E>  // bf16 or fp16 rows
__device__ __forceinline__ __amdgpu_buffer_rsrc_t chunk_rows_rsrc(E* base, int start, int len, int H, int h) {
  return __builtin_amdgcn_make_buffer_rsrc(base + ((size_t)start * H + h) * D, (short)0, (len - 1) * H * D * 2 + D * 2,
                                           0x00020000);
}
// a raw buffer resource over ``bytes`` bytes from ``base``
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}
__device__ __forceinline__ void buf_stf(__amdgpu_buffer_rsrc_t rs, int voff, int soff, float x) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, x), rs, voff, soff, 0);
}
template <class X8>
__device__ __forceinline__ void buf_st16(__amdgpu_buffer_rsrc_t rs, int voff, int soff, X8 x) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, x), rs, voff, soff, 0);
}
__device__ __forceinline__ void buf_st1(__amdgpu_buffer_rsrc_t rs, int voff, int soff, float x) {
  __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, (bf16)x), rs, voff, soff, 0);
}
// four values rounded to E (bf16 or fp16), 8 bytes
template <class E = bf16>
__device__ __forceinline__ void buf_st4(__amdgpu_buffer_rsrc_t rs, int voff, int soff, f32x4 x) {
  __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, to4<E>(x)), rs, voff, soff, 0);
}

// ---- hand-off between two kernels running at the same time ----------------
// The eight XCDs' L2 caches are not coherent with one another.  Data that one
// running kernel hands to another is stored and loaded with the cache-policy bit
// sc1 (device scope), as relaxed agent-scope atomics are: the store writes
// through to the device-coherent level, and the load does not take a line that
// another XCD may have changed.  The count announcing the data is an agent-scope
// atomic add, issued only after the data's stores have completed (vmcnt), and
// read with an agent-scope load before any of the data is loaded.
constexpr int CPOL_NT = 2, CPOL_SC1 = 16;  // aux bits of the buffer and load-to-LDS intrinsics (gfx950)
__device__ __forceinline__ void dma16_sc1(const void* src, void* lds) {
  __builtin_amdgcn_global_load_lds(src, (lds_void_ptr)lds, 16, 0, CPOL_SC1);
}
template <class X8>
__device__ __forceinline__ X8 buf_ld16_sc1(__amdgpu_buffer_rsrc_t rs, int voff) {
  return __builtin_bit_cast(X8, __builtin_amdgcn_raw_buffer_load_b128(rs, voff, 0, CPOL_SC1));
}
// 16 bytes stored at device scope with the non-temporal hint
template <class X8>
__device__ __forceinline__ void buf_st16_nt_sc1(__amdgpu_buffer_rsrc_t rs, int voff, X8 x) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, x), rs, voff, 0, CPOL_NT | CPOL_SC1);
}
__device__ __forceinline__ void count_add(int* p) {
  __hip_atomic_fetch_add(p, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int count_read(const int* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Poll *p until it reaches target, sleeping about 8,000 cycles (a few
// microseconds) between polls: hundreds of waiting workgroups polling a few
// lines faster than that slow the scan they wait for (a lone waiter may poll
// faster: SLEEP is s_sleep's argument, in units of 64 cycles).  Bounded: false
// after `limit` polls (COUNT_SPIN_LIMIT: about a second), so a hand-off that
// never comes ends the waiting kernel with poisoned results instead of hanging it.
constexpr int COUNT_SPIN_LIMIT = 1 << 18;
template <int SLEEP = 127>
__device__ __forceinline__ bool count_wait_ge(const int* p, int target, int limit = COUNT_SPIN_LIMIT) {
  for (int i = 0; i < limit; ++i) {
    if (count_read(p) >= target) return true;
    __builtin_amdgcn_s_sleep(SLEEP);
  }
  return false;
}

// Per-chunk metadata: chunk_table[c] = (start event, length).  A chunk never
// crosses a document boundary; doc_chunk[d] .. doc_chunk[d+1] are the chunks of
// document d, in time order.
struct ChunkInfo {
  int start, len;
};
__device__ __forceinline__ ChunkInfo chunk_info(const int32_t* table, int c) {
  return ChunkInfo{table[2 * c], table[2 * c + 1]};
}

// The (head, chunk position) of this workgroup in a grid of (H, NC) chunk-heads.
// The dispatcher deals consecutive workgroups out to the XCDs in turn, so with the
// plain mapping (head = blockIdx.x) each XCD holds H / 8 heads of every chunk, and
// each line of an fp32 [T][H] array (g, beta, the norms, dg: 128 bytes = two events of
// all 16 heads) is fetched into all eight L2s.  Here the j-th workgroup an XCD receives
// takes head j % H of chunk position 8 (j / H) + xcd: all heads of a chunk run on one
// XCD, at about the same time, and share those lines in its L2.  Positions still come
// in blocks of eight chunks in dispatch order; the last NC % 8 positions keep the plain
// mapping.  A bijection of [0, H NC) for any H, NC.  Below kXcdMapMinChunks chunks the
// plain mapping is kept: those arrays are then small, and at 36 chunks (config 1) the
// mapping made the step 1% slower where at 144 it made it 1% faster.
constexpr int kXcds = 8, kXcdMapMinChunks = 64;
struct HeadChunk {
  int h, p;
};
__device__ __forceinline__ HeadChunk xcd_head_chunk(int H, int NC) {
  const int i = blockIdx.y * gridDim.x + blockIdx.x;  // dispatch order
  const int full = NC / kXcds * kXcds;
  if (NC >= kXcdMapMinChunks && i < full * H) {
    const int xcd = i % kXcds, j = i / kXcds;
    return HeadChunk{j % H, j / H * kXcds + xcd};
  }
  return HeadChunk{i % H, i / H};
}

}  // namespace cqgdn
