"""GPU parity of the HIP GDN kernels against the CPU oracle (float64), through the C ABI.

Cases follow the reference's NPU gates: lengths 1/63/64/65/129/257 with packed
documents (scripts/validation/delta_ascendc_validate.py:21-27), intermediates
gcum / T / w / u / h / v_new (scripts/validation/delta_ascendc_diagnose.py:23-42),
read-only bit-exactness (tests/test_qwen35_cq.py:71-89) and document isolation
(tests/test_document_packing.py:180-200).
"""

import pytest
import torch

from gdn_testlib import (TOL_BF16, TOL_INTER, TOL_STATE, assemble, assert_close_bf16, compare_layer, layer_parity, perm32,
                         rel_l2, view)
from oracle import gdn_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def inputs(T, H, seed, readonly=None):
    from cqgdn import synthetic

    return synthetic.make_inputs(T, H, 128, seed=seed, readonly=readonly)


def to_dev(xs):
    return [x.to(DEV) for x in xs]


def run_fwd(gdn, xs, bounds, training=True, want_state=False, normalize=True, initial_state=None):
    q, k, v, g, b = to_dev(xs)
    o, state, ws = gdn._forward(q, k, v, g.contiguous(), b.contiguous(), bounds, normalize, 128 ** -0.5,
                                training=training, want_state=want_state, initial_state=initial_state)
    torch.cuda.synchronize()
    return o, state, ws


CASES = [
    (1, (0, 1), 4),
    (63, (0, 63), 4),
    (64, (0, 64), 4),
    (65, (0, 65), 4),
    (129, (0, 129), 16),
    (129, (0, 37, 129), 16),
    (257, (0, 1, 37, 64, 200, 257), 8),
    # 4 and 5 chunks: the scans' first stage refill and their last copy-outs meet
    (256, (0, 256), 4),
    (300, (0, 300), 4),
]


@pytest.mark.parametrize("T,bounds,H", CASES)
def test_forward_intermediates_and_output(gdn, T, bounds, H):
    print(f"case T={T} bounds={bounds} H={H}", flush=True)
    check_forward(gdn, T, bounds, H, seed=900 + T)


# 102 and 146 chunks: from 64 chunks on the chunk kernels map all heads of a chunk to one
# XCD in blocks of eight chunk positions, and the last 6 (resp. 2) positions keep the
# plain mapping; every chunk-head's intermediates are checked
@pytest.mark.parametrize("T,bounds,H", [(6454, (0, 3000, 6454), 16), (9300, (0, 9300), 16)])
def test_forward_xcd_mapped_chunks(gdn, T, bounds, H):
    print(f"case T={T} bounds={bounds} H={H}", flush=True)
    check_forward(gdn, T, bounds, H, seed=T)


def check_forward(gdn, T, bounds, H, seed):
    """The forward's output and stored intermediates against the oracle's."""
    xs = inputs(T, H, seed=seed)
    o, _, ws = run_fwd(gdn, xs, bounds)
    q, k, v, g, b = (x.double() for x in xs)
    ref, inter = O.chunk_delta(q, k, v, g, b, bounds, return_intermediates=True)
    from cqgdn import _lib

    spans = inter["spans"]
    nc = len(spans)
    off = _lib.fwd_offsets(T, H, nc)
    gc = view(ws, off["gcum"], torch.float32, (T, H))
    assert rel_l2(gc, assemble(inter["gcum"], spans, T)) < 1e-6
    Tm = view(ws, off["T"], torch.bfloat16, (nc, H, 64, 64))
    W = view(ws, off["W"], torch.bfloat16, (T, H, 128))
    UT = view(ws, off["UT"], torch.bfloat16, (nc, H, 128, 64))
    hT = view(ws, off["hT"], torch.bfloat16, (nc, H, 128, 128))
    vnT = view(ws, off["vnT"], torch.bfloat16, (nc, H, 128, 64))
    for c, (a, e) in enumerate(spans):
        n = e - a
        assert rel_l2(Tm[c, :, :n, :n], inter["T"][c]) < TOL_INTER
        assert rel_l2(UT[c, :, :, :n].transpose(-1, -2), inter["U"][c]) < TOL_INTER
        # h is exactly zero on the first chunk of every document
        assert rel_l2(hT[c].transpose(-1, -2), inter["h"][c]) < TOL_INTER
        assert rel_l2(vnT[c, :, :, :n].transpose(-1, -2), inter["vn"][c]) < TOL_INTER
        # rows past the tail are zero (the scan relies on it for U, the backward for v_new)
        assert float(UT[c, :, :, n:].abs().max() if n < 64 else 0) == 0.0
        assert float(vnT[c, :, :, n:].abs().max() if n < 64 else 0) == 0.0
    # W is stored in perm32 column order (logical column x at perm32(x))
    perm = torch.tensor([perm32(x) for x in range(128)])
    assert rel_l2(-W[..., perm], assemble(inter["W"], spans, T)) < TOL_INTER  # stored negated
    assert_close_bf16("o", o.cpu(), ref)


@pytest.mark.parametrize("T,bounds,H", CASES)
def test_backward_matches_oracle(gdn, T, bounds, H):
    print(f"case T={T} bounds={bounds} H={H}", flush=True)
    xs = inputs(T, H, seed=1900 + T)
    gen = torch.Generator().manual_seed(7 + T)
    do = torch.randn(1, T, H, 128, generator=gen).bfloat16()
    xd = [x.to(DEV).requires_grad_() for x in xs]
    cu = torch.tensor(bounds, device=DEV)
    y, _ = gdn.delta(*xd, use_qk_l2norm_in_kernel=True, cu_seqlens=cu, cu_seqlens_cpu=torch.tensor(bounds))
    y.backward(do.to(DEV))
    torch.cuda.synchronize()
    q, k, v, g, b = (x.double() for x in xs)
    ref = O.chunk_delta(q, k, v, g, b, bounds)
    grads = O.chunk_delta_backward(q, k, v, g, b, do.double(), bounds)
    assert_close_bf16("o", y.detach().cpu(), ref)
    for name, x, r in zip(("dq", "dk", "dv", "dg", "dbeta"), xd, grads):
        assert x.grad.dtype == x.dtype
        assert_close_bf16(name, x.grad.cpu(), r)


def test_backward_intermediates(gdn):
    T, H, bounds = 200, 4, (0, 70, 200)
    xs = inputs(T, H, seed=5)
    gen = torch.Generator().manual_seed(11)
    do = torch.randn(1, T, H, 128, generator=gen).bfloat16()
    do_dev = do.to(DEV)
    from cqgdn import _lib

    q, k, v, g, b = to_dev(xs)
    o, _, ws = gdn._forward(q, k, v, g, b, bounds, True, 128 ** -0.5, training=True)
    _, table, doc = gdn.device_metadata(bounds, DEV)
    nc = table.shape[0]
    bws = torch.empty(_lib.lib().cqgdn_bwd_workspace_size(T, H, nc), dtype=torch.uint8, device=DEV)
    dq, dk, dv = (torch.empty_like(v) for _ in range(3))
    dg, db = torch.empty_like(g), torch.empty_like(b)
    P = gdn._ptr
    gdn.call("cqgdn_bwd", P(q), P(k), P(v), P(g), P(b), P(do_dev), T, H, P(table), nc, P(doc), len(bounds) - 1,
             128 ** -0.5, 3, P(ws), ws.numel(), P(bws), bws.numel(), P(dq), P(dk), P(dv), P(dg), P(db),
             gdn._stream(q.device))
    torch.cuda.synchronize()
    qd, kd, vd, gd, bd = (x.double() for x in xs)
    _, binter = O.chunk_delta_backward(qd, kd, vd, gd, bd, do.double(), bounds, return_intermediates=True)
    off = _lib.bwd_offsets(T, H, nc)
    dvlT = view(bws, off["dvlT"], torch.bfloat16, (nc, H, 128, 64))
    XT = view(bws, off["XT"], torch.bfloat16, (nc, H, 128, 128))
    # value-slice-major dh [8][k][16] and dv_new [8][t][16] -> (k, v) and (t, v)
    dh = view(bws, off["dh"], torch.bfloat16, (nc, H, 8, 128, 16)).permute(0, 1, 3, 2, 4).reshape(nc, H, 128, 128)
    dVn = view(bws, off["dVn"], torch.bfloat16, (nc, H, 8, 64, 16)).permute(0, 1, 3, 2, 4).reshape(nc, H, 64, 128)
    spans = O.chunk_spans(bounds)
    for c, (a, e) in enumerate(spans):
        n = e - a
        assert rel_l2(dvlT[c, :, :, :n].transpose(-1, -2), binter["dv_local"][c]) < TOL_INTER, c
        assert rel_l2(XT[c].transpose(-1, -2), binter["X"][c]) < TOL_INTER, c
        if binter["dh"][c].abs().max() > 0:
            assert rel_l2(dh[c], binter["dh"][c]) < TOL_INTER, c
        assert rel_l2(dVn[c, :, :n], binter["dVn"][c]) < 2 * TOL_INTER, c
        assert not dVn[c, :, n:].any(), c  # rows past the tail are zero (bwd_dkw reads them unmasked)


def test_cq_config1_shape_fwd_bwd(gdn):
    """Config 1 event stream (2048 content + 256 read-only after it), H=16, fwd+bwd vs the oracle."""
    from cqgdn import synthetic

    T, mask, bounds = synthetic.config_events(1, seed=1)
    xs = inputs(T, 16, seed=1, readonly=mask)
    gen = torch.Generator().manual_seed(101)
    do = torch.randn(1, T, 16, 128, generator=gen).bfloat16()
    xd = [x.to(DEV).requires_grad_() for x in xs]
    y, _ = gdn.delta(*xd, use_qk_l2norm_in_kernel=True)
    y.backward(do.to(DEV))
    torch.cuda.synchronize()
    q, k, v, g, b = (x.double() for x in xs)
    assert_close_bf16("o", y.detach().cpu(), O.chunk_delta(q, k, v, g, b))
    grads = O.chunk_delta_backward(q, k, v, g, b, do.double())
    for name, x, r in zip(("dq", "dk", "dv", "dg", "dbeta"), xd, grads):
        assert_close_bf16(name, x.grad.cpu(), r)


def test_readonly_events_leave_state_and_outputs_bit_identical(gdn):
    """Perturbing read-only queries changes nothing but their own outputs (tests/test_qwen35_cq.py:71-89)."""
    from cqgdn import synthetic

    T = 640
    mask = synthetic.cq_readonly_mask(512, 2, 64, seed=4)
    xs = inputs(T, 8, seed=3, readonly=mask)
    o1, s1, _ = run_fwd(gdn, xs, (0, T), training=False, want_state=True)
    q2 = xs[0].clone()
    q2[:, mask] = (q2[:, mask].float() * 10 + 3).bfloat16()
    o2, s2, _ = run_fwd(gdn, [q2, *xs[1:]], (0, T), training=False, want_state=True)
    assert torch.equal(o1[:, ~mask.to(DEV)], o2[:, ~mask.to(DEV)])
    assert torch.equal(s1, s2)
    # removing the read-only events entirely gives the same final state
    keep = ~mask
    o3, s3, _ = run_fwd(gdn, [x[:, keep] for x in xs], (0, int(keep.sum())), training=False, want_state=True)
    assert rel_l2(s3, s1) < TOL_STATE


@pytest.mark.parametrize("training", [True, False])
def test_documents_are_isolated(gdn, training):
    """Changing document A leaves document B bit-identical (tests/test_document_packing.py:180-200):
    the outputs of the training forward, and outputs and final states of the inference forward."""
    bounds = (0, 150, 301, 400)
    xs = inputs(400, 8, seed=21)
    o1, s1, _ = run_fwd(gdn, xs, bounds, training=training, want_state=not training)
    changed = [x.clone() for x in xs]
    changed[0][:, :150] += 1
    changed[2][:, :150] *= 3
    changed[3][:, :150] -= 0.5
    o2, s2, _ = run_fwd(gdn, changed, bounds, training=training, want_state=not training)
    assert torch.equal(o1[:, 150:], o2[:, 150:])
    if not training:
        assert torch.equal(s1[1:], s2[1:])
    assert not torch.equal(o1[:, :150], o2[:, :150])


def test_prefill_final_state_and_initial_state(gdn):
    """prefill() runs the precise (fp16-operand) forward: final states within 1e-3 of the float64 oracle."""
    T, H, bounds = 300, 16, (0, 100, 300)
    xs = inputs(T, H, seed=31)
    q, k, v, g, b = to_dev(xs)
    o, state = gdn.prefill(q, k, v, g, b, bounds)
    torch.cuda.synchronize()
    qd, kd, vd, gd, bd = (x.double() for x in xs)
    ref, ref_state = O.chunk_delta(qd, kd, vd, gd, bd, bounds, output_final_state=True)
    assert_close_bf16("o", o.cpu(), ref)
    r = rel_l2(state, ref_state)
    print(f"  final state rel_l2={r:.3e}", flush=True)
    assert r <= TOL_STATE
    # continuing from a state: prefill(a ++ b) == prefill(b, initial_state=prefill(a))
    s0 = torch.randn(1, H, 128, 128, generator=torch.Generator().manual_seed(3)) * 0.02
    o4, st4 = gdn.prefill(q[:, 100:], k[:, 100:], v[:, 100:], g[:, 100:], b[:, 100:], (0, 200),
                          initial_state=s0.to(DEV))
    ref4, rst4 = O.chunk_delta(qd[:, 100:], kd[:, 100:], vd[:, 100:], gd[:, 100:], bd[:, 100:], (0, 200),
                               initial_state=s0.double(), output_final_state=True)
    assert_close_bf16("o(initial_state)", o4.cpu(), ref4)
    r4 = rel_l2(st4, rst4)
    print(f"  final state (initial_state) rel_l2={r4:.3e}", flush=True)
    assert r4 <= TOL_STATE


@pytest.mark.parametrize("v_scale,s0_scale", [(300.0, 0.0), (1e-3, 0.0), (1.0, 500.0), (1e4, 1e4)])
def test_prefill_precise_range_scaling(gdn, v_scale, s0_scale):
    """The precise forward scales V (and the initial state) by a power of two to keep its fp16
    operands in range: results stay within tolerance for values far from 1, with no inf/nan."""
    T, H, bounds = 200, 4, (0, 70, 200)
    print(f"case v_scale={v_scale} s0_scale={s0_scale}", flush=True)
    q, k, v, g, b = inputs(T, H, seed=61)
    v = (v.float() * v_scale).bfloat16()
    s0 = torch.randn(2, H, 128, 128, generator=torch.Generator().manual_seed(62)) * s0_scale
    o, state = gdn.prefill(*to_dev([q, k, v, g, b]), bounds, initial_state=s0.to(DEV) if s0_scale else None)
    torch.cuda.synchronize()
    assert torch.isfinite(o.float()).all() and torch.isfinite(state).all()
    ref, ref_state = O.chunk_delta(q.double(), k.double(), v.double(), g.double(), b.double(), bounds,
                                   initial_state=s0.double() if s0_scale else None, output_final_state=True)
    assert_close_bf16("o", o.cpu(), ref)
    r = rel_l2(state, ref_state)
    print(f"  final state rel_l2={r:.3e}", flush=True)
    assert r <= TOL_STATE


def test_config2_full_size_fwd_bwd(gdn):
    """Config 2 at full size (8192 content + 4x256 read-only at seeded positions, H=16), fwd+bwd vs the oracle."""
    from cqgdn import synthetic

    T, mask, bounds = synthetic.config_events(2, seed=0)
    print(f"case config 2 T={T}", flush=True)
    xs = inputs(T, 16, seed=2, readonly=mask)
    do = torch.randn(1, T, 16, 128, generator=torch.Generator().manual_seed(102)).bfloat16()
    xd = [x.to(DEV).requires_grad_() for x in xs]
    y, _ = gdn.delta(*xd, use_qk_l2norm_in_kernel=True)
    y.backward(do.to(DEV))
    torch.cuda.synchronize()
    q, k, v, g, b = (x.double() for x in xs)
    assert_close_bf16("o", y.detach().cpu(), O.chunk_delta(q, k, v, g, b))
    grads = O.chunk_delta_backward(q, k, v, g, b, do.double())
    for name, x, r in zip(("dq", "dk", "dv", "dg", "dbeta"), xd, grads):
        assert_close_bf16(name, x.grad.cpu(), r)


def test_config3_packed_documents_fwd_bwd_and_states(gdn):
    """Config 3: 32768 events in seeded documents of 256..4096 (last truncated), state reset per document."""
    from cqgdn import synthetic

    T, _, bounds = synthetic.config_events(3, seed=0)
    print(f"case config 3 T={T} docs={len(bounds) - 1}", flush=True)
    xs = inputs(T, 16, seed=3)
    do = torch.randn(1, T, 16, 128, generator=torch.Generator().manual_seed(103)).bfloat16()
    xd = [x.to(DEV).requires_grad_() for x in xs]
    cu = torch.tensor(bounds, device=DEV)
    y, _ = gdn.delta(*xd, use_qk_l2norm_in_kernel=True, cu_seqlens=cu, cu_seqlens_cpu=list(bounds))
    y.backward(do.to(DEV))
    _, states = gdn.prefill(*[x.detach() for x in xd], bounds)
    torch.cuda.synchronize()
    q, k, v, g, b = (x.double() for x in xs)
    ref, ref_states = O.chunk_delta(q, k, v, g, b, bounds, output_final_state=True)
    assert_close_bf16("o", y.detach().cpu(), ref)
    grads = O.chunk_delta_backward(q, k, v, g, b, do.double(), bounds)
    for name, x, r in zip(("dq", "dk", "dv", "dg", "dbeta"), xd, grads):
        assert_close_bf16(name, x.grad.cpu(), r)
    worst = max(rel_l2(states[d], ref_states[d]) for d in range(len(bounds) - 1))
    print(f"  worst per-document final state rel_l2={worst:.3e}", flush=True)
    assert worst <= TOL_STATE


@pytest.mark.parametrize("E,beta_bf16", [(1, False), (2, False), (2, True), (5, False)])
def test_recurrent_decode_step(gdn, E, beta_bf16):
    N, H = 6, 16
    gen = torch.Generator().manual_seed(40 + E)
    q = O.l2norm(torch.randn(N, E, H, 128, generator=gen)).bfloat16()
    k = O.l2norm(torch.randn(N, E, H, 128, generator=gen)).bfloat16()
    v = torch.randn(N, E, H, 128, generator=gen).bfloat16()
    g = -torch.nn.functional.softplus(torch.randn(N, E, H, generator=gen))
    b = torch.randn(N, E, H, generator=gen).sigmoid()
    if E == 2:  # the CQ decode buffer: event 1 is a read-only query
        k[:, 1] = 0
        v[:, 1] = 0
        g[:, 1] = 0
        b[:, 1] = 0
    if beta_bf16:
        b = b.bfloat16()
    state = torch.randn(N, H, 128, 128, generator=gen) * 0.02
    ref_state = state.double().clone()
    ref = O.decode_step(q.double(), k.double(), v.double(), g.double(), b.double(), ref_state)
    st = state.to(DEV)
    ptr = st.data_ptr()
    out = torch.empty(N, E, H, 128, dtype=torch.bfloat16, device=DEV)
    gdn.recurrent(q.to(DEV), k.to(DEV), v.to(DEV), g.to(DEV), b.to(DEV), st, out)
    torch.cuda.synchronize()
    assert st.data_ptr() == ptr
    assert_close_bf16("o", out.cpu(), ref)
    r = rel_l2(st, ref_state)
    print(f"  state rel_l2={r:.3e}", flush=True)
    assert r <= TOL_STATE


def test_recurrent_reference_call_shape(gdn):
    """The reference's call: q [t,H,128], state [1,H,V,K] (ops/gated_delta_net.py:321-351)."""
    H = 8
    gen = torch.Generator().manual_seed(9)
    q = O.l2norm(torch.randn(2, H, 128, generator=gen)).bfloat16()
    k = O.l2norm(torch.randn(2, H, 128, generator=gen)).bfloat16()
    v = torch.randn(2, H, 128, generator=gen).bfloat16()
    g = -torch.rand(2, H, generator=gen)
    b = torch.rand(2, H, generator=gen).bfloat16()
    state = torch.randn(1, H, 128, 128, generator=gen) * 0.1
    ref_state = state.double().clone()
    ref = O.decode_step(q[None].double(), k[None].double(), v[None].double(), g[None].double(), b[None].double(),
                        ref_state)[0]
    st, out = state.to(DEV), torch.empty(2, H, 128, dtype=torch.bfloat16, device=DEV)
    gdn.recurrent(q.to(DEV), k.to(DEV), v.to(DEV), g.to(DEV), b.to(DEV), st, out)
    torch.cuda.synchronize()
    assert_close_bf16("o", out.cpu(), ref)
    assert rel_l2(st, ref_state) <= TOL_STATE


def test_l2norm_and_cumsum_kernels(gdn):
    gen = torch.Generator().manual_seed(2)
    x = torch.randn(37, 3, 128, generator=gen).bfloat16()
    y, rstd = gdn.l2_fwd(x.to(DEV))
    assert_close_bf16("l2_fwd", y.cpu(), O.l2norm(x.double()))
    dy = torch.randn(37, 3, 128, generator=gen).bfloat16()
    xx = x.double().requires_grad_()
    O.l2norm(xx).backward(dy.double())
    assert_close_bf16("l2_bwd", gdn.l2_bwd(y, rstd, dy.to(DEV)).cpu(), xx.grad)
    g = torch.randn(1, 300, 4, generator=gen)
    bounds = (0, 10, 200, 300)
    # the reference's head-first layout [B, H, T] (ops/gated_delta_net.py:77-87, :204)
    out = gdn.reverse_cumsum(g.transpose(1, 2).contiguous().to(DEV), bounds)
    ref = O.chunk_local_cumsum(g.double(), bounds, reverse=True)
    assert out.shape == (1, 4, 300)
    assert rel_l2(out.transpose(1, 2), ref) < 1e-6
    # unpacked batch: every row its own sequence
    g2 = torch.randn(3, 4, 130, generator=gen)
    out2 = gdn.reverse_cumsum(g2.to(DEV), None)
    ref2 = torch.stack([O.chunk_local_cumsum(g2[i].T[None].double(), (0, 130), reverse=True)[0].T for i in range(3)])
    assert rel_l2(out2, ref2) < 1e-6


def test_forward_backward_bitwise_deterministic(gdn):
    from cqgdn import synthetic

    T, mask, bounds = synthetic.config_events(1, seed=2)
    xs = inputs(T, 16, seed=2, readonly=mask)
    do = torch.randn(1, T, 16, 128, generator=torch.Generator().manual_seed(3)).bfloat16().to(DEV)
    outs = []
    for _ in range(2):
        xd = [x.to(DEV).requires_grad_() for x in xs]
        y, _ = gdn.delta(*xd, use_qk_l2norm_in_kernel=True)
        y.backward(do)
        outs.append([y.detach()] + [x.grad for x in xd])
    torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert torch.equal(a, b)


def test_whole_layer_matches_oracle_recurrence(gdn):
    """The GatedDelta layer mirror (width 2048, image-CQ plan) run by the fused kernels
    (events.layer_core) against the same bf16 layer run by the reference's torch code whose
    recurrence is the float64 CPU oracle: output, dx and the input-projection gradient (the
    quantities the reference's layer benchmark compares, scripts/benchmark_gdn.py:58-63)."""
    import layer_harness as layer

    print("case whole layer: content 300, 120 queries, image groups (40, 24)", flush=True)
    torch.manual_seed(5)
    model = layer.GatedDeltaLayer().to(DEV, torch.bfloat16)
    model.A_log.data = model.A_log.data.float()
    model.norm_weight.data = model.norm_weight.data.float()
    plan = layer.cq_layer_plan(300, 120, image_groups=(40, 24), seed=3).to(DEV)
    gen = torch.Generator().manual_seed(6)
    x = torch.randn(plan.hidden_length, 1, 2048, generator=gen).bfloat16().to(DEV)
    up = (torch.randn(plan.hidden_length, 1, 2048, generator=gen) / 100).bfloat16().to(DEV)

    def run(recurrence):
        model.zero_grad(set_to_none=True)
        xx = x.clone().requires_grad_()
        y = model(xx, plan, recurrence=recurrence)
        (y * up).sum().backward()
        torch.cuda.synchronize()
        return y.detach().float().cpu(), xx.grad.float().cpu(), model.in_proj_all.weight.grad.float().cpu()

    def oracle(q, k, v, g, b, p):
        ins = [t.detach().double().cpu().requires_grad_() for t in (q, k, v, g, b)]
        out = O.recurrent_delta(*ins, p.event_bounds, normalize=True)

        class Bridge(torch.autograd.Function):  # float64 CPU recurrence inside the bf16 GPU graph
            @staticmethod
            def forward(ctx, *dev_ins):
                return out.detach().to(q.device, q.dtype)

            @staticmethod
            def backward(ctx, dy):
                grads = torch.autograd.grad(out, ins, dy.double().cpu())
                return tuple(gr.to(t.device, t.dtype) for gr, t in zip(grads, (q, k, v, g, b)))

        return Bridge.apply(q, k, v, g, b)

    got, want = run(None), run(oracle)
    for name, a, b in zip(("y", "dx", "dW_in"), got, want):
        assert_close_bf16(name, a, b.double())


@pytest.mark.parametrize("T,C,K,bounds,act", [
    (1, 64, 4, (0, 1), True),
    (37, 64, 4, (0, 1, 3, 37), True),
    (75, 64, 3, (0, 40, 75), True),
    (200, 128, 2, (0, 200), False),
    (1000, 256, 4, (0, 5, 64, 65, 96, 97, 600, 1000), True),
    (300, 6144, 4, (0, 2, 130, 131, 300), True),
    (5000, 512, 4, (0, 1234, 1235, 5000), True),  # 40-row strips of the backward
    (3001, 256, 3, (0, 3001), True),  # strips of 24 rows, K = 3 groups
])
def test_conv1d_matches_oracle(gdn, T, C, K, bounds, act):
    """Packed causal conv1d (fwd, dx, dw) against the float64 oracle: documents of 1-2 rows,
    row tiles crossing documents, the layer's 6144 channels, K = 2..4, with and without SiLU."""
    print(f"case conv T={T} C={C} K={K} bounds={bounds} act={act}", flush=True)
    gen = torch.Generator().manual_seed(T * 31 + C + K)
    x = torch.randn(1, T, C, generator=gen).bfloat16()
    w = (torch.randn(C, K, generator=gen) * 0.5).bfloat16()
    dy = torch.randn(1, T, C, generator=gen).bfloat16()
    xd, wd = x.to(DEV).requires_grad_(), w.to(DEV).requires_grad_()
    cu = torch.tensor(bounds, dtype=torch.int32, device=DEV)
    y, _ = gdn.conv(xd, wd, activation="silu" if act else None, cu_seqlens=cu, cu_seqlens_cpu=bounds)
    y.backward(dy.to(DEV))
    torch.cuda.synchronize()
    xr, wr = x.double().requires_grad_(), w.double().requires_grad_()
    yr = O.causal_conv1d(xr, wr, bounds, activation=act)
    yr.backward(dy.double())
    assert_close_bf16("y", y.detach().cpu(), yr.detach())
    assert_close_bf16("dx", xd.grad.cpu(), xr.grad)
    assert_close_bf16("dw", wd.grad.cpu(), wr.grad)
    assert wd.grad.dtype == torch.bfloat16


def test_conv1d_deterministic_and_unpacked(gdn):
    """The conv backward is bitwise deterministic (fixed-order dw reduction); an unpacked batch
    treats every row as its own document."""
    gen = torch.Generator().manual_seed(1)
    x = torch.randn(3, 50, 64, generator=gen).bfloat16().to(DEV)
    w = torch.randn(64, 4, generator=gen).bfloat16().to(DEV)
    dy = torch.randn(3, 50, 64, generator=gen).bfloat16().to(DEV)
    outs = []
    for _ in range(2):
        xd, wd = x.clone().requires_grad_(), w.clone().requires_grad_()
        y, _ = gdn.conv(xd, wd, activation="silu")
        y.backward(dy)
        outs.append((y.detach(), xd.grad, wd.grad))
    torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    yr = O.causal_conv1d(x.cpu().double(), w.cpu().double(), None)
    assert_close_bf16("y unpacked", outs[0][0].cpu(), yr)


@pytest.mark.parametrize("fused", [False, True])
def test_gated_norm_matches_oracle(gdn, fused):
    """The gated RMSNorm against the float64 oracle and its autograd: plain, and fused with a
    row gather (padding rows -1, y rows no row reads, z a column slice of a wider projection)."""
    gen = torch.Generator().manual_seed(21 + fused)
    H, y_rows = 4, 50
    y = torch.randn(y_rows, H, 128, generator=gen).bfloat16()
    w = (1 + 0.2 * torch.randn(128, generator=gen)).float()
    if fused:
        perm = torch.randperm(y_rows, generator=gen)[:37]
        index = torch.cat((perm[:20], torch.tensor([-1, -1]), perm[20:])).to(torch.int32)
        rows = index.numel()
        proj = torch.randn(rows, 3 * H * 128 + 40, generator=gen).bfloat16()
        z = proj[:, H * 128:2 * H * 128].reshape(rows, H, 128)  # strided rows
    else:
        index, rows = None, y_rows
        z = torch.randn(y_rows, H, 128, generator=gen).bfloat16()
    dout = torch.randn(rows, H, 128, generator=gen).bfloat16()
    yd, wd = y.to(DEV).requires_grad_(), w.to(DEV).requires_grad_()
    zsrc = (proj if fused else z).to(DEV).requires_grad_()
    zd = zsrc[:, H * 128:2 * H * 128].reshape(rows, H, 128) if fused else zsrc
    out = gdn.gated_norm(yd, zd, wd, index=index.to(DEV) if fused else None)
    out.backward(dout.to(DEV))
    torch.cuda.synchronize()
    yr, zr, wr = y.double().requires_grad_(), z.double().requires_grad_(), w.double().requires_grad_()
    if fused:
        gathered = torch.where((index >= 0)[:, None, None], yr[index.clamp(min=0).long()], torch.zeros_like(yr[:1]))
    else:
        gathered = yr
    ref = O.gated_rms_norm(gathered, zr, wr)
    ref.backward(dout.double())
    assert_close_bf16("out", out.detach().cpu(), ref.detach())
    assert_close_bf16("dy", yd.grad.cpu(), yr.grad)
    dz = zsrc.grad.cpu()
    if fused:
        assert dz[:, :H * 128].abs().max() == 0 and dz[:, 2 * H * 128:].abs().max() == 0
        dz = dz[:, H * 128:2 * H * 128].reshape(rows, H, 128)
        unread = sorted(set(range(y_rows)) - set(index[index >= 0].tolist()))
        assert yd.grad[unread].abs().max().item() == 0  # rows no one reads get zero gradients
    assert_close_bf16("dz", dz, zr.grad)
    assert_close_bf16("dweight", wd.grad.cpu(), wr.grad)


def test_gated_norm_backward_deterministic(gdn):
    """Two backward passes of the fused gated norm are bitwise equal (fixed-order dweight)."""
    gen = torch.Generator().manual_seed(5)
    y = torch.randn(3000, 16, 128, generator=gen).bfloat16().to(DEV)
    z = torch.randn(3000, 16, 128, generator=gen).bfloat16().to(DEV)
    w = torch.randn(128, generator=gen).to(DEV)
    dout = torch.randn(3000, 16, 128, generator=gen).bfloat16().to(DEV)
    grads = []
    for _ in range(2):
        yd, zd, wd = y.clone().requires_grad_(), z.clone().requires_grad_(), w.clone().requires_grad_()
        gdn.gated_norm(yd, zd, wd).backward(dout)
        grads.append((yd.grad, zd.grad, wd.grad))
    torch.cuda.synchronize()
    for a, b in zip(*grads):
        assert torch.equal(a, b)


@pytest.mark.parametrize("seed", range(4))
@pytest.mark.parametrize("docs", [1, 2])
def test_layer_core_matches_float64_restatement(gdn, docs, seed):
    """events.layer_core (conv over gathered rows, query conv, event gathers and gates, the
    recurrence, output gather and gated norm, and their inverse-map backward) against the
    reference's layer code in float64 on the CPU with the oracle conv, recurrence and norm, from
    the same bf16 projection: output rows and the gradients of the projection (every column:
    q|k|v, z, a, b), the conv weight, A_log, dt_bias (conditioned control error) and the norm weight."""
    import layer_harness as layer

    print(f"case layer core: {docs} document(s), seed {seed}", flush=True)
    if docs == 1:
        plan = layer.cq_layer_plan(300, 90, image_groups=(40, 24), seed=4)
    else:
        plan = layer.concat_plans(layer.cq_layer_plan(200, 50, image_groups=(30,), seed=5),
                                  layer.cq_layer_plan(150, 40, image_groups=(20, 10), seed=6))
    H, S = 16, 2048
    gen = torch.Generator().manual_seed(40 + docs + 1000 * seed)
    proj = (torch.randn(plan.hidden_length, 4 * S + 2 * H, generator=gen) * 0.7).bfloat16()
    compare_layer(*layer_parity(plan, proj, H, gen), H)


def _decode_params(gen, H, K=4):
    S = H * 128
    w = (torch.rand(3 * S, K, generator=gen) - 0.5).bfloat16()
    A_log = torch.rand(H, generator=gen).mul(3).add(0.01).log()
    dt_bias = torch.randn(H, generator=gen) * 0.5
    nw = 1 + 0.1 * torch.randn(128, generator=gen)
    return w, A_log, dt_bias, nw


def test_layer_decode_step_matches_oracle(gdn):
    """Three consecutive decode steps (models/decoding.py:16-78) of three sequences through
    cqgdn_layer_decode_step against the float64 oracle step: the gated-norm rows of C and Q, the
    conv history (bit-exact: it holds raw rows) and the value-first state."""
    from cqgdn import events

    print("case layer decode: N=3, H=16, K=4, 3 steps", flush=True)
    gen = torch.Generator().manual_seed(61)
    N, H, K = 3, 16, 4
    S, P = H * 128, 4 * H * 128 + 2 * H
    w, A_log, dt_bias, nw = _decode_params(gen, H, K)
    hist = (torch.randn(N, K - 1, 3 * S, generator=gen) * 0.7).bfloat16()
    state = torch.randn(N, H, 128, 128, generator=gen) * 0.05
    cache = {"conv": hist.to(DEV), "state": state.to(DEV)}
    ref_hist, ref_state = hist.double(), state.double()
    dev = [t.to(DEV) for t in (w, A_log, dt_bias, nw)]
    for step in range(3):
        proj = (torch.randn(N, 2, P, generator=gen) * 0.7).bfloat16()
        out = events.layer_decode_step(proj.to(DEV), *dev, cache, heads=H)
        torch.cuda.synchronize()
        args = (proj[..., :3 * S], proj[..., 3 * S:4 * S].reshape(N, 2, H, 128), proj[..., 4 * S:4 * S + H],
                proj[..., 4 * S + H:], w, A_log, dt_bias, nw)
        ref_out, ref_hist, ref_state = O.layer_decode_step(*args, ref_hist, ref_state)
        assert_close_bf16(f"out step {step}", out.cpu(), ref_out.reshape(N, 2, S))
        assert torch.equal(cache["conv"].cpu().double(), ref_hist), "conv history differs"
        assert_close_bf16(f"state step {step}", cache["state"].cpu(), ref_state)


def test_layer_prefill_then_decode_matches_one_shot(gdn):
    """Prefill with the uncommitted target (the CQDecoder convention, models/decoding.py:117-121),
    then one decode step, equals the one-shot prefill of the plan where the step's content token
    commits and its query reads after it: the C and Q rows and the final state, through two
    independent routes (chunked precise forward vs the streaming decode step)."""
    from cqgdn import events
    from gdn_testlib import decode_plans

    print("case prefill -> decode: 150 content rows, H=16", flush=True)
    gen = torch.Generator().manual_seed(62)
    n, H, K = 150, 16, 4
    S, P = H * 128, 4 * H * 128 + 2 * H
    w, A_log, dt_bias, nw = (t.to(DEV) for t in _decode_params(gen, H, K))
    pre_plan, one_plan = decode_plans(n, K)
    proj = (torch.randn(n + 2, P, generator=gen) * 0.7).bfloat16().to(DEV)
    _, cache = events.layer_prefill(proj[:n + 1], w, A_log, dt_bias, nw, pre_plan, heads=H)
    assert torch.equal(cache["conv"][0], proj[n - K + 1:n, :3 * S])
    out = events.layer_decode_step(proj[n:n + 2], w, A_log, dt_bias, nw, cache, heads=H)
    one, one_cache = events.layer_prefill(proj, w, A_log, dt_bias, nw, one_plan, heads=H)
    torch.cuda.synchronize()
    assert_close_bf16("C and Q rows", out.cpu(), one[n:n + 2].double().cpu())
    assert_close_bf16("state", cache["state"].cpu(), one_cache["state"].double().cpu())
    assert torch.equal(cache["conv"][0], proj[n - K + 2:n + 1, :3 * S])
