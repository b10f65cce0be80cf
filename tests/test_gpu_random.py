"""Seeded random sweep of the drop-in path against the float64 oracle on the GPU.

Each case draws a head count the reference accepts (ops/gated_delta_net.py:235), packed
documents with empty, one-event, partial-chunk, whole-chunk and multi-chunk lengths
(host_bounds allows empty documents, ops/gated_delta_net.py:102-114), a share of read-only
CQ events (k = v = g = beta = 0, tests/test_qwen35_cq.py), the in-kernel l2norm on or off and
both backward modes, then compares the output and all five gradients with the oracle
(the reference's NPU gate: relative L2 within 2e-2).  The fp16 cases draw the same kinds of
batches with fp16 q/k/v and dO (the fp16 kernels, CQGDN_FP16) and hold them to TOL_FP16.  The
prefill cases add random initial states and compare the per-document final states to 1e-3.
The long cases (at least 64 chunks, up to about 11,000 events in one to three documents) run
the chunk kernels' XCD-aware mapping and, in the cached mode, bwd_dkw beside the reverse scan.
"""

import random

import pytest
import torch

from gdn_testlib import TOL_BF16, TOL_FP16, TOL_STATE, assert_close_bf16, rel_l2
from oracle import gdn_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def draw_case(seed):
    rnd = random.Random(seed)
    H = rnd.choice([4, 8, 16, 32])
    lens = [rnd.choice([0, 1, rnd.randint(2, 63), 64, rnd.randint(65, 200), rnd.randint(201, 420)])
            for _ in range(rnd.randint(1, 5))]
    if sum(lens) == 0:
        lens[-1] = rnd.randint(1, 100)
    bounds = [0]
    for n in lens:
        bounds.append(bounds[-1] + n)
    return H, tuple(bounds), rnd.choice([0.0, 0.0, 0.25]), rnd.random() < 0.75, rnd.choice(["cached", "fused"])


def make(T, H, seed, readonly_share, normalize, dtype=torch.bfloat16):
    from cqgdn import synthetic

    gen = torch.Generator().manual_seed(7000 + seed)
    readonly = (torch.rand(T, generator=gen) < readonly_share) if readonly_share else None
    q, k, v, g, b = synthetic.make_inputs(T, H, 128, seed=8000 + seed, readonly=readonly, dtype=dtype)
    if not normalize:  # callers that normalize themselves pass unit rows (zero rows stay zero)
        q, k = (O.l2norm(x.double()).to(dtype) for x in (q, k))
    return [q, k, v, g, b]


def _training_case(gdn, monkeypatch, seed, dtype, tol):
    H, bounds, ro, normalize, mode = draw_case(seed)
    T = bounds[-1]
    print(f"case seed={seed} T={T} bounds={bounds} H={H} readonly={ro} normalize={normalize} mode={mode} "
          f"{dtype}", flush=True)
    monkeypatch.setattr(gdn, "MODE", mode)
    xs = make(T, H, seed, ro, normalize, dtype)
    do = torch.randn(1, T, H, 128, generator=torch.Generator().manual_seed(9000 + seed)).to(dtype)
    xd = [x.to(DEV).requires_grad_() for x in xs]
    cu = torch.tensor(bounds, device=DEV)
    y, _ = gdn.delta(*xd, use_qk_l2norm_in_kernel=normalize, cu_seqlens=cu, cu_seqlens_cpu=list(bounds))
    y.backward(do.to(DEV))
    torch.cuda.synchronize()
    assert y.dtype == dtype and all(x.grad.dtype == x.dtype for x in xd)
    q, k, v, g, b = (x.double() for x in xs)
    assert_close_bf16("o", y.detach().cpu(), O.chunk_delta(q, k, v, g, b, bounds, normalize=normalize), tol=tol)
    ref = O.chunk_delta_backward(q, k, v, g, b, do.double(), bounds, normalize=normalize)
    for name, x, r in zip(("dq", "dk", "dv", "dg", "dbeta"), xd, ref):
        assert_close_bf16(name, x.grad.cpu(), r, tol=tol)


@pytest.mark.parametrize("seed", range(12))
def test_random_training_case_matches_oracle(gdn, monkeypatch, seed):
    _training_case(gdn, monkeypatch, seed, torch.bfloat16, TOL_BF16)


@pytest.mark.parametrize("seed", range(200, 208))
def test_random_fp16_training_case_matches_oracle(gdn, monkeypatch, seed):
    _training_case(gdn, monkeypatch, seed, torch.float16, TOL_FP16)


@pytest.mark.parametrize("seed", range(100, 106))
def test_random_prefill_case_matches_oracle(gdn, seed):
    H, bounds, ro, _, _ = draw_case(seed)
    T, n_docs = bounds[-1], len(bounds) - 1
    print(f"case prefill seed={seed} T={T} bounds={bounds} H={H} readonly={ro}", flush=True)
    xs = make(T, H, seed, ro, True)
    s0 = 0.02 * torch.randn(n_docs, H, 128, 128, generator=torch.Generator().manual_seed(9500 + seed))
    o, states = gdn.prefill(*[x.to(DEV) for x in xs], bounds, initial_state=s0.to(DEV))
    torch.cuda.synchronize()
    q, k, v, g, b = (x.double() for x in xs)
    ref_o, ref_states = O.chunk_delta(q, k, v, g, b, bounds, initial_state=s0.double(), output_final_state=True)
    assert_close_bf16("o", o.cpu(), ref_o)
    for d in range(n_docs):
        r = rel_l2(states[d].cpu(), ref_states[d])
        assert r <= TOL_STATE, f"document {d} (length {bounds[d + 1] - bounds[d]}): final state rel_l2 {r:.3e}"


def draw_long_case(seed):
    """4, 8 or 16 heads; one to three documents of 2,000 to 11,000 events, so that every batch has
    at least 64 chunks (the chunk kernels then put all heads of a chunk on one XCD, and bwd_dkw runs
    beside the reverse scan where it fits); cached or fused mode; bf16 or fp16."""
    rnd = random.Random(seed)
    H = rnd.choice([4, 8, 16])
    n_docs = rnd.randint(1, 3)
    lens = [rnd.randint(2000, 9000 // n_docs + 2000) for _ in range(n_docs)]
    bounds = [0]
    for n in lens:
        bounds.append(bounds[-1] + n)
    return H, tuple(bounds), rnd.choice(["cached", "fused"]), rnd.choice([torch.bfloat16, torch.float16])


@pytest.mark.parametrize("seed", range(3000, 3008))
def test_random_long_case_matches_oracle(gdn, monkeypatch, seed):
    H, bounds, mode, dtype = draw_long_case(seed)
    T = bounds[-1]
    print(f"case long seed={seed} T={T} bounds={bounds} H={H} mode={mode} {dtype}", flush=True)
    monkeypatch.setattr(gdn, "MODE", mode)
    tol = TOL_FP16 if dtype == torch.float16 else TOL_BF16
    xs = make(T, H, seed, 0.2, True, dtype)
    do = torch.randn(1, T, H, 128, generator=torch.Generator().manual_seed(9000 + seed)).to(dtype)
    xd = [x.to(DEV).requires_grad_() for x in xs]
    y, _ = gdn.delta(*xd, use_qk_l2norm_in_kernel=True, cu_seqlens=torch.tensor(bounds, device=DEV),
                     cu_seqlens_cpu=list(bounds))
    y.backward(do.to(DEV))
    torch.cuda.synchronize()
    q, k, v, g, b = (x.double() for x in xs)
    assert_close_bf16("o", y.detach().cpu(), O.chunk_delta(q, k, v, g, b, bounds), tol=tol)
    ref = O.chunk_delta_backward(q, k, v, g, b, do.double(), bounds)
    for name, x, r in zip(("dq", "dk", "dv", "dg", "dbeta"), xd, ref):
        assert_close_bf16(name, x.grad.cpu(), r, tol=tol)
