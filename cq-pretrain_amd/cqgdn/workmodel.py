"""Algorithmic work of each libcqgdn kernel: FLOPs and HBM bytes per launch.

FLOPs are the minimal GEMM set of the chunked WY form, per (chunk of c events,
head), d = d_k = d_v = 128:

  forward  10 c^2 d + 6 c d^2 + (2/3) c^3
           (beta K K^T, W, U, Q K^T, P v_new; W S, Q S, K^T v_new; UT inverse)
  backward 20 c^2 d + 12 c d^2 + 4 c^3   (recompute not counted)

split over the kernels by the contractions each one performs:

  fwd_prep   beta K K^T, W = T (beta gamma K), U = T (beta V), UT inverse   6 c^2 d + (2/3) c^3
  fwd_scan   W S, K^T v_new                                                 4 c d^2
  fwd_out    Q S, Q K^T, P v_new                                            2 c d^2 + 4 c^2 d
  bwd_local  dv_local = P^T dO, X = Q^T dO (P and -W^T recomputed, not counted)  2 c^2 d + 2 c d^2
  bwd_scan   dS += W^T dv_new, dv_new += Kg dS                              4 c d^2
  bwd_dkw    dP, dQ and dK from P, dQ from S, dK from dS, dW = -dv_new S^T;
             dT (2), d(beta gamma K), d(beta V), dA = -T^T dT T^T, dK from dA  18 c^2 d + 6 c d^2 + 4 c^3

HBM bytes are the kernel's declared inputs and outputs, each read or written
once, in the workspace layouts of gdn_layout.hpp: event-indexed rows scale with
the events of the chunk, chunk-indexed tiles ([D][64], [64][64], [D][D]) are
stored whole.  Traffic counters above these figures mean re-reads.

The decode step (``recurrent``) moves per sequence and head, per event:
read + write of the fp32 state (2 d^2 4 B), q, k, v (3 d 2 B), g and beta
(2 x 4 B) and the output (d 2 B).
"""

from __future__ import annotations

D = 128
CHUNK = 64
PEAK_BF16_FLOPS = 2.5e15  # MI355X dense bf16 MFMA
PEAK_HBM_BYTES = 8.0e12  # MI355X HBM3E

FWD_KERNELS = ("fwd_prep", "fwd_scan", "fwd_out")
BWD_KERNELS = ("bwd_local", "bwd_scan", "bwd_dkw")
SCAN_KERNELS = ("fwd_scan", "bwd_scan")


def chunk_lengths(bounds, chunk=CHUNK):
    """Lengths of every chunk of the packed documents ``bounds`` (0, ..., T)."""
    out = []
    for a, b in zip(bounds, bounds[1:]):
        out.extend(min(chunk, b - s) for s in range(a, b, chunk))
    return out


def flops_per_chunk(kernel, c, d=D):
    """Algorithmic FLOPs of one (chunk of c events, head) in ``kernel``."""
    c2d, cd2, c3 = c * c * d, c * d * d, c ** 3
    return {
        "fwd_prep": 6 * c2d + 2 * c3 / 3,
        "fwd_scan": 4 * cd2,
        "fwd_out": 2 * cd2 + 4 * c2d,
        "bwd_local": 2 * c2d + 2 * cd2,
        "bwd_scan": 4 * cd2,
        "bwd_dkw": 18 * c2d + 6 * cd2 + 4 * c3,
    }[kernel]


def bytes_per_chunk(kernel, c, d=D):
    """Algorithmic HBM bytes of one (chunk of c events, head) in ``kernel``."""
    e = c * d * 2  # bf16 event rows of the chunk
    e32 = c * d * 4  # fp32 event rows
    s = c * 4  # fp32 per-event scalars
    tile = CHUNK * d * 2  # bf16 [D][64] chunk tile
    sq = d * d * 2  # bf16 [D][D] chunk state
    tm = CHUNK * CHUNK * 2  # bf16 [64][64] T matrix
    return {
        # k,v,g,beta -> rk,gcum,T,-W rows,U^T,KgT (q's l2 scale is formed by its readers)
        "fwd_prep": 2 * e + 2 * s + 2 * s + tm + e + 2 * tile,
        # -W rows, U^T, KgT, gcum -> h^T, v_new^T
        "fwd_scan": e + 2 * tile + s + sq + tile,
        # q, k, rk, gcum, h^T, v_new^T -> o
        "fwd_out": 2 * e + 2 * s + sq + tile + e,
        # q, k, rk, dO, gcum, beta, T -> dv_local^T, X^T, kdec Kn perm32, -W^T
        "bwd_local": 3 * e + 3 * s + tm + tile + sq + e + tile,
        # kdec Kn perm32, gcum, dv_local^T, X^T, -W^T -> dh, dv_new (both value-slice-major)
        "bwd_scan": e + s + tile + sq + tile + sq + tile,
        # q, k, rk, gcum, h^T, v_new^T, dO, dh, dv_new, v, beta, T -> dq, dk, dv, dg, dbeta
        "bwd_dkw": 2 * e + 2 * s + sq + tile + e + sq + tile + e + s + tm + 3 * e + 2 * s,
    }[kernel]


def kernel_work(kernel, bounds, heads):
    """(FLOPs, bytes) of one launch of ``kernel`` over packed ``bounds`` with ``heads`` heads."""
    lengths = chunk_lengths(bounds)
    flops = heads * sum(flops_per_chunk(kernel, c) for c in lengths)
    nbytes = heads * sum(bytes_per_chunk(kernel, c) for c in lengths)
    return flops, nbytes


def decode_bytes(n_seq, heads, events=1, d=D):
    """HBM bytes of one ``recurrent`` launch over n_seq sequences of ``events`` events."""
    per = 2 * d * d * 4 + events * (3 * d * 2 + 2 * 4 + d * 2)
    return n_seq * heads * per
