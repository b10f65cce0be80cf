"""Seeded synthetic GDN workloads of the benchmark configurations.

Distributions follow the benchmark definition: q, k, v ~ N(0,1) (bf16),
beta = sigmoid(N(0,1)), g = -softplus(N(0,1)) (fp32 [1,T,H]).  Read-only CQ
query events carry a real q and k = v = 0, g = beta = 0, which is how the
reference's layer builds them (models/backbone_qwen35.py:184-194).
"""

from __future__ import annotations

import torch
from torch.nn import functional as F


def cq_readonly_mask(content: int, blocks: int, block_len: int = 256, *, seed: int = 0, after: bool = False):
    """Event mask [content + blocks*block_len], True on read-only query events.

    ``after``: all query blocks follow the content (config 1); otherwise the
    blocks are inserted at seeded, sorted content positions (config 2).
    """
    total = content + blocks * block_len
    mask = torch.zeros(total, dtype=torch.bool)
    if blocks == 0:
        return mask
    if after:
        mask[content:] = True
        return mask
    gen = torch.Generator().manual_seed(seed)
    cuts = sorted(torch.randint(0, content + 1, (blocks,), generator=gen).tolist())
    at = 0
    for i, cut in enumerate(cuts):
        start = cut + i * block_len
        mask[start:start + block_len] = True
        at = start + block_len
    assert int(mask.sum()) == blocks * block_len and at <= total
    return mask


def doc_bounds(total: int, lo: int = 256, hi: int = 4096, *, seed: int = 3):
    """Packed document bounds (0, ..., total) with lengths ~ U[lo, hi], last one truncated."""
    gen = torch.Generator().manual_seed(seed)
    bounds = [0]
    while bounds[-1] < total:
        n = int(torch.randint(lo, hi + 1, (1,), generator=gen))
        bounds.append(min(total, bounds[-1] + n))
    return tuple(bounds)


def make_inputs(T: int, H: int = 16, D: int = 128, *, seed: int = 0, readonly=None, device="cpu",
                dtype=torch.bfloat16):
    """q, k, v [1,T,H,D] (``dtype``) and g, beta [1,T,H] fp32, generated on the CPU then moved."""
    gen = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(1, T, H, D, generator=gen).to(dtype) for _ in range(3))
    beta = torch.randn(1, T, H, generator=gen).sigmoid()
    g = -F.softplus(torch.randn(1, T, H, generator=gen))
    if readonly is not None:
        m = torch.as_tensor(readonly, dtype=torch.bool)
        k[:, m] = 0
        v[:, m] = 0
        g[:, m] = 0
        beta[:, m] = 0
    return tuple(x.to(device) for x in (q, k, v, g, beta))


def config_events(config: int, *, seed: int = 0):
    """(T, readonly mask or None, bounds) of benchmark configs 0..3 (H=16, d=128)."""
    if config == 0:
        return 2048, None, (0, 2048)
    if config == 1:
        m = cq_readonly_mask(2048, 1, 256, seed=seed, after=True)
        return m.numel(), m, (0, m.numel())
    if config == 2:
        m = cq_readonly_mask(8192, 4, 256, seed=seed)
        return m.numel(), m, (0, m.numel())
    if config == 3:
        b = doc_bounds(32768, seed=seed + 3)
        return 32768, None, b
    raise ValueError(f"no event stream for config {config}")
