// Workspace layout of the GDN forward/backward passes (host and device).
//
// In the precise forward (CQGDN_PRECISE) and with fp16 inputs (CQGDN_FP16) every
// buffer listed as bf16 holds fp16, in the scales the kernels state (V's s_v for
// U, h and v_new; dO's s_d for the backward's buffers).
//
// The forward workspace holds everything the backward re-reads apart from the
// inputs (the reference saves q,k,v,gcum,beta,A in fused mode and also
// w,h,v_new in cached mode, ops/gated_delta_net.py:184); keeping h and v_new
// avoids re-running the serial state scan in the backward.  No normalized copy
// of q and k is kept: every reader scales its q and k rows by their l2 scales on
// the way into LDS, with the rounding fwd_prep applies (bf16 or fp16 of
// float(x) * r).  The k scales rk are kept; the q scales are formed by each
// kernel that reads q rows (row_rnorm), so no kernel before them reads q.
// Buffers are addressed by event (time-first [T][H][D], the caller's TND
// order) or by chunk ([NC][H][...], one 64-event block per chunk, rows past a
// tail chunk's length are zero).  Value-slice-major
// buffers ([8][rows][16]: slice s holds values 16 s .. 16 s + 15 of every row)
// are written by the state scans, whose workgroups each own one 16-wide value
// slice: a scan step stores one contiguous block, and a reader's MFMA fragment
// (8 consecutive values of one row) is one contiguous 16-byte load.
#pragma once
#include <stddef.h>
#include <stdint.h>

namespace cqgdn {

enum FwdBuf {
  F_RK = 0,  // f32  [T][H]      rsqrt(sum k^2 + eps) (1 without the in-kernel l2norm)
  F_GC,      // f32  [T][H]      chunk-local cumsum of g
  F_TM,      // bf16 [NC][H][64][64]  T = (I + A)^-1, row-major (t, s)
  F_W,       // bf16 [T][H][D]   -W, W = T (beta*exp(G)*K), rows (t, k), perm32 column order
  F_UT,      // bf16 [NC][H][D][64]   U = T (beta*V) transposed (v, t)
  F_KGT,     // bf16 [NC][H][D][64]   (K * exp(G_last - G)) transposed (k, t), perm32 columns
  F_HT,      // bf16 [NC][H][D][D]    state entering the chunk, (v, k)
  F_VNT,     // bf16 [NC][H][D][64]   v_new transposed (v, t)
  F_VSC,     // f32  [1 + 1024]       power-of-two scale s_v of V and block partials (fp16 operands)
  F_COUNT
};

enum BwdBuf {
  B_DVLT = 0,  // bf16 [NC][H][D][64]  local dv = scale*P^T dO, (v, t)
  B_XT,        // bf16 [NC][H][D][D]   X = scale*(gam*Qn)^T dO, (v, k)
  B_DH,        // bf16 [NC][H][8][D][16]  gradient of the state leaving the chunk, value-slice-major (s, k, v%16)
  B_DVN,       // bf16 [NC][H][8][64][16] d v_new, value-slice-major (s, t, v%16)
  B_KNP,       // bf16 [T][H][D]       exp(G_last - G_t) Kn_t in perm32 column order (reverse scan operand), by bwd_local
  B_WT,        // bf16 [NC][H][D][64]  -W transposed (k, t), perm32 column order (reverse scan operand), by bwd_local
  B_SYNC,      // i32  [NC][H] + 64     per (chunk, head): reverse-scan value slices whose dS / dVn are stored,
               //                       then at [NC][H] the count of resident reverse-scan workgroups
               //                       (bwd_dkw beside the scan; zeroed by bwd_local)
  B_DSC,       // f32  [1 + 1024]       power-of-two scale s_d of dO and block partials (fp16 operands)
  B_COUNT
};

constexpr size_t kAlign = 256;
constexpr int kVscaleBlocks = 1024;  // partial maxima behind the fp16 paths' scales of V and dO
// the scales bring max|V| (and the initial state) into [2^(t-1), 2^t): t for inference, and
// for training, where the backward also keeps products of V- and dO-scaled values in fp16
constexpr int kVscaleTarget = 6, kVscaleTargetTraining = 3;

inline size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

inline void fwd_sizes(int64_t T, int64_t H, int64_t NC, size_t* s) {
  const size_t ev = (size_t)T * H, chunk = (size_t)NC * H;
  s[F_RK] = ev * 4;
  s[F_GC] = ev * 4;
  s[F_TM] = chunk * 64 * 64 * 2;
  s[F_W] = ev * 128 * 2;
  s[F_UT] = chunk * 128 * 64 * 2;
  s[F_KGT] = chunk * 128 * 64 * 2;
  s[F_HT] = chunk * 128 * 128 * 2;
  s[F_VNT] = chunk * 128 * 64 * 2;
  s[F_VSC] = (1 + kVscaleBlocks) * 4;
}

inline void bwd_sizes(int64_t T, int64_t H, int64_t NC, size_t* s) {
  const size_t ev = (size_t)T * H, chunk = (size_t)NC * H;
  s[B_DVLT] = chunk * 128 * 64 * 2;
  s[B_XT] = chunk * 128 * 128 * 2;
  s[B_DH] = chunk * 128 * 128 * 2;
  s[B_DVN] = chunk * 64 * 128 * 2;
  s[B_KNP] = ev * 128 * 2;
  s[B_WT] = chunk * 128 * 64 * 2;
  s[B_SYNC] = (chunk + 64) * 4;
  s[B_DSC] = (1 + kVscaleBlocks) * 4;
}

// Offsets of every buffer; returns the total size in bytes.
inline size_t offsets(const size_t* sizes, int n, size_t* off) {
  size_t at = 0;
  for (int i = 0; i < n; ++i) {
    off[i] = at;
    at += align_up(sizes[i]);
  }
  return at;
}

}  // namespace cqgdn
