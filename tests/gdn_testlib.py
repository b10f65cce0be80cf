"""Helpers shared by the GPU parity tests: error metrics and workspace views."""

from __future__ import annotations

import torch

# Tolerances (written here and used by every parity test):
#  * bf16 outputs and gradients vs the float64 oracle: relative-L2 <= 2e-2 and
#    normalized max error max|a-b| / max|b| <= 2e-2
#  * fp32 final states: relative-L2 <= 1e-3
#  * read-only events / other documents: bit-identical (atol = rtol = 0)
TOL_BF16 = 2e-2
TOL_STATE = 1e-3
TOL_INTER = 1e-2  # bf16-rounded intermediates (T, W, U, h, v_new, ...)


def rel_l2(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def max_rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))


def assert_close_bf16(name, actual, expected, tol=TOL_BF16):
    assert torch.isfinite(actual.float()).all(), f"{name}: non-finite values"
    r, m = rel_l2(actual, expected), max_rel(actual, expected)
    print(f"  {name}: rel_l2={r:.3e} max_rel={m:.3e}", flush=True)
    assert r <= tol and m <= tol, f"{name}: rel_l2={r:.3e} max_rel={m:.3e} > {tol}"


def view(ws, offset, dtype, shape):
    n = 1
    for s in shape:
        n *= s
    nbytes = n * torch.tensor([], dtype=dtype).element_size()
    return ws[offset:offset + nbytes].view(dtype).view(*shape)


def assemble(chunks, spans, T):
    """Per-chunk oracle tensors [H, n, ...] -> time-first [T, H, ...]."""
    first = chunks[0]
    out = first.new_zeros(T, first.shape[0], *first.shape[2:])
    for x, (a, b) in zip(chunks, spans):
        out[a:b] = x.transpose(0, 1)
    return out


def perm32(x):
    """Storage position of logical column x in the kernels' perm32 order (gdn_common.hpp)."""
    return (x & ~31) | (((x >> 2) & 3) << 3) | (((x >> 4) & 1) << 2) | (x & 3)


def decode_plans(n, kernel=4):
    """Plans of a single document for the prefill -> decode invariant (models/decoding.py:105-121).

    ``prefill``: content rows 0..n, each a single-token group written by its own event, except
    row n, the uncommitted target (read-only event), as CQDecoder prepares its prefill.
    ``one_shot``: the same rows with row n written (the decode step's C) and one CQ query read
    after it (the decode step's Q, hidden row n + 1), whose conv history is rows n-K+2 .. n.
    """
    from cqgdn import layer

    long = lambda xs: torch.tensor(xs, dtype=torch.long)

    def make(writes_last, query):
        nc = n + 1
        eq, ew = list(range(nc)), list(range(n)) + [n if writes_last else nc]
        qs, qh, hidden = [], [], list(range(nc))
        if query:
            eq.append(nc)
            ew.append(nc)
            qs, qh = [nc], [list(range(n - kernel + 2, n + 1))]
            hidden.append(nc)
        return layer.LayerPlan(
            content_order=torch.arange(nc), event_q=long(eq), event_write=long(ew), query_source=long(qs),
            query_history=long(qh).reshape(len(qs), kernel - 1), content_cu=torch.tensor([0, nc], dtype=torch.int32),
            content_bounds=(0, nc), event_cu=long([0, len(eq)]), event_bounds=(0, len(eq)),
            hidden_length=len(hidden), hidden_event=long(hidden))

    return make(False, False), make(True, True)
