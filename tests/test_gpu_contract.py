"""GPU parity of contract shapes the reference accepts, through the public API against the oracle.

* ``delta`` at H = 32, the largest local head count of ops/gated_delta_net.py:235, and the fused
  layer and its decode step at H = 32;
* packed batches holding empty documents (host_bounds allows b == a, ops/gated_delta_net.py:112):
  outputs, gradients, and prefill final states (an empty document's state is its initial state);
* config 4 at its own shape: 64 sequences, H = 16, fp32 state, 256 consecutive ``recurrent``
  steps against the float64 oracle step (models/decoding.py:71-77);
* the CQ read-only invariant of tests/test_qwen35_cq.py:71-89, bit-exact, on the bf16 training
  path of ``delta`` and through ``events.layer_core``: perturbed query rows leave every content
  output bit-identical, a perturbed image group leaves every output read before the group's first
  write bit-identical, and an image group's outputs see its last token;
* the fused layer on plans whose content rows share hidden rows (the two-branch Bi_I+CQ_T plans
  of ops/gated_delta_layout.py:66-83), and on a projection that is a column slice of a wider tensor.
"""

import numpy as np
import pytest
import torch

from gdn_testlib import TOL_BF16, TOL_FP16, TOL_STATE, assert_close_bf16, compare_layer, layer_parity, rel_l2, view
from oracle import gdn_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def inputs(T, H, seed, readonly=None):
    from cqgdn import synthetic

    return synthetic.make_inputs(T, H, 128, seed=seed, readonly=readonly)


def fwd_bwd(gdn, xs, bounds, do):
    xd = [x.to(DEV).requires_grad_() for x in xs]
    kw = {}
    if bounds is not None:
        kw = dict(cu_seqlens=torch.tensor(bounds, device=DEV), cu_seqlens_cpu=list(bounds))
    y, _ = gdn.delta(*xd, use_qk_l2norm_in_kernel=True, **kw)
    y.backward(do.to(DEV))
    torch.cuda.synchronize()
    return y.detach().cpu(), [x.grad.cpu() for x in xd]


def check_against_oracle(xs, bounds, do, y, grads):
    q, k, v, g, b = (x.double() for x in xs)
    assert_close_bf16("o", y, O.chunk_delta(q, k, v, g, b, bounds))
    ref = O.chunk_delta_backward(q, k, v, g, b, do.double(), bounds)
    for name, x, r in zip(("dq", "dk", "dv", "dg", "dbeta"), grads, ref):
        assert_close_bf16(name, x, r)


@pytest.mark.parametrize("T,bounds", [(200, (0, 70, 200)), (130, None)])
def test_delta_h32_matches_oracle(gdn, T, bounds):
    """H = 32 (ops/gated_delta_net.py:235): fwd+bwd against the float64 oracle."""
    print(f"case H=32 T={T} bounds={bounds}", flush=True)
    xs = inputs(T, 32, seed=3200 + T)
    do = torch.randn(1, T, 32, 128, generator=torch.Generator().manual_seed(32)).bfloat16()
    y, grads = fwd_bwd(gdn, xs, bounds, do)
    check_against_oracle(xs, bounds, do, y, grads)


@pytest.mark.parametrize("bounds", [(0, 0, 130, 257), (0, 0, 130, 130, 257, 257), (0, 64, 64, 65)])
def test_packed_batch_with_empty_documents(gdn, bounds):
    """Empty documents (b == a in the bounds) at the start, middle and end of a packed batch."""
    T, H = bounds[-1], 8
    print(f"case empty documents bounds={bounds}", flush=True)
    xs = inputs(T, H, seed=77 + len(bounds))
    do = torch.randn(1, T, H, 128, generator=torch.Generator().manual_seed(78)).bfloat16()
    y, grads = fwd_bwd(gdn, xs, bounds, do)
    check_against_oracle(xs, bounds, do, y, grads)
    # prefill: per-document final states; an empty document's state is its initial state
    n_docs = len(bounds) - 1
    s0 = torch.randn(n_docs, H, 128, 128, generator=torch.Generator().manual_seed(79)) * 0.05
    for init in (None, s0):
        _, states = gdn.prefill(*[x.to(DEV) for x in xs], bounds,
                                initial_state=None if init is None else init.to(DEV))
        torch.cuda.synchronize()
        q, k, v, g, b = (x.double() for x in xs)
        _, ref_states = O.chunk_delta(q, k, v, g, b, bounds, output_final_state=True,
                                      initial_state=None if init is None else init.double())
        for d, (a, e) in enumerate(zip(bounds, bounds[1:])):
            if a == e:
                want = torch.zeros(H, 128, 128) if init is None else init[d]
                assert torch.equal(states[d].cpu(), want), f"empty document {d} changed its state"
            else:
                r = rel_l2(states[d], ref_states[d])
                print(f"  document {d} final state rel_l2={r:.3e}", flush=True)
                assert r <= TOL_STATE


def test_config4_decode_256_steps_matches_oracle(gdn):
    """Config 4 at its own shape: B = 64 sequences, H = 16, fp32 state [64,16,128,128] ~ N(0, 0.02),
    q/k l2-normalised bf16, beta = sigmoid(N(0,1)), g = -softplus(N(0,1)), 256 consecutive
    ``recurrent`` steps against the float64 oracle step.  Every step's output within the bf16 bar,
    the state within 1e-3 (fp32) after the last step."""
    N, H, steps = 64, 16, 256
    print(f"case config 4: N={N} H={H} steps={steps}", flush=True)
    gen = torch.Generator().manual_seed(4)
    state0 = torch.randn(N, H, 128, 128, generator=gen) * 0.02
    st = state0.to(DEV)
    ins, outs = [], []
    for step in range(steps):
        q = O.l2norm(torch.randn(N, 1, H, 128, generator=gen)).bfloat16()
        k = O.l2norm(torch.randn(N, 1, H, 128, generator=gen)).bfloat16()
        v = torch.randn(N, 1, H, 128, generator=gen).bfloat16()
        b = torch.randn(N, 1, H, generator=gen).sigmoid()
        g = -torch.nn.functional.softplus(torch.randn(N, 1, H, generator=gen))
        out = torch.empty(N, 1, H, 128, dtype=torch.bfloat16, device=DEV)
        gdn.recurrent(q.to(DEV), k.to(DEV), v.to(DEV), g.to(DEV), b.to(DEV), st, out)
        ins.append((q, k, v, g, b))
        outs.append(out)
    torch.cuda.synchronize()
    print("  gpu steps done", flush=True)
    ref_state = state0.double()
    worst = 0.0
    for step, ((q, k, v, g, b), out) in enumerate(zip(ins, outs)):
        ref = O.decode_step(q.double(), k.double(), v.double(), g.double(), b.double(), ref_state)
        r = rel_l2(out, ref)
        worst = max(worst, r)
        assert r <= TOL_BF16, f"step {step}: output rel_l2={r:.3e}"
    rs = rel_l2(st, ref_state)
    print(f"  worst output rel_l2={worst:.3e}, final state rel_l2={rs:.3e}", flush=True)
    assert rs <= TOL_STATE


def test_cq_invariant_bf16_training_delta(gdn):
    """tests/test_qwen35_cq.py:71-77 on the bf16 training path: perturbing the read-only query
    rows (q * 10 + noise) leaves every content output bit-identical; the gradients still flow."""
    from cqgdn import synthetic

    mask = synthetic.cq_readonly_mask(2048, 1, 256, seed=5)  # one query block inside the content
    T = mask.numel()
    print(f"case CQ invariant, training delta, T={T}", flush=True)
    xs = inputs(T, 16, seed=55, readonly=mask)
    do = torch.randn(1, T, 16, 128, generator=torch.Generator().manual_seed(56)).bfloat16()
    y1, _ = fwd_bwd(gdn, xs, None, do)
    q2 = xs[0].clone()
    noise = torch.randn(q2[:, mask].shape, generator=torch.Generator().manual_seed(57))
    q2[:, mask] = (q2[:, mask].float() * 10 + noise * 10).bfloat16()
    y2, g2 = fwd_bwd(gdn, [q2, *xs[1:]], None, do)
    assert torch.equal(y1[:, ~mask], y2[:, ~mask])
    assert not torch.equal(y1[:, mask], y2[:, mask])
    assert all(torch.isfinite(g.float()).all() for g in g2)


def _layer_params(H, gen):
    S = H * 128
    w = (torch.rand(3 * S, 4, generator=gen) - 0.5).bfloat16()
    A_log = torch.rand(H, generator=gen).mul(3).add(0.01).log()
    dt_bias = torch.randn(H, generator=gen) * 0.5
    nw = 1 + 0.1 * torch.randn(128, generator=gen)
    return [t.to(DEV) for t in (w, A_log, dt_bias, nw)]


def test_cq_invariant_layer_core(gdn):
    """tests/test_qwen35_cq.py:71-89 through the fused layer (events.layer_core): query rows
    perturbed by N(0,1) * 10 leave every content row bit-identical; an image group perturbed the
    same way leaves every row whose output event precedes the group's first write bit-identical
    (the queries of earlier or equal sigma and the content before it); the group's first image
    output sees its last token."""
    from cqgdn import events
    import layer_harness as layer

    H, S = 16, 2048
    plan = layer.cq_layer_plan(600, 160, image_groups=(64, 40), seed=8).to(DEV)
    print(f"case CQ invariant, layer_core: {plan.hidden_length} rows", flush=True)
    gen = torch.Generator().manual_seed(81)
    params = _layer_params(H, gen)
    proj = (torch.randn(plan.hidden_length, 4 * S + 2 * H, generator=gen) * 0.7).bfloat16()
    n_c = plan.content_order.numel()

    def run(p):
        with torch.no_grad():
            out = events.layer_core(p.to(DEV), *params, plan, heads=H)
        torch.cuda.synchronize()
        return out.cpu()

    base = run(proj)
    changed = proj.clone()
    changed[n_c:] += (torch.randn(changed[n_c:].shape, generator=gen) * 10).bfloat16()
    after = run(changed)
    assert torch.equal(base[:n_c], after[:n_c])
    assert not torch.equal(base[n_c:], after[n_c:])
    # the second image group (content rows written as one multi-token group)
    ew, hidden = plan.event_write.cpu(), plan.hidden_event.cpu()
    rows = _image_group_rows(plan, size=40)
    first_write = int(torch.nonzero(torch.isin(ew, rows)).min())
    keep = hidden < first_write
    assert int(keep.sum()) > 100 and bool(keep[n_c:].any())  # content and queries on both sides
    changed = proj.clone()
    changed[rows] += (torch.randn(changed[rows].shape, generator=gen) * 10).bfloat16()
    after = run(changed)
    assert torch.equal(base[keep], after[keep])
    assert not torch.equal(base[~keep], after[~keep])
    changed = proj.clone()
    changed[rows[-1]] += (torch.randn(changed[rows[-1]].shape, generator=gen) * 3).bfloat16()
    after = run(changed)
    assert float((base[rows[0]].float() - after[rows[0]].float()).abs().max()) > 1e-8


def _image_group_rows(plan, size):
    """Hidden rows of the multi-token group of ``size`` members: each such group's members are
    read again right after the group is written, so its re-reads are one run of consecutive
    events (runs of two groups are separated by the second group's writes)."""
    ew, eq = plan.event_write.cpu(), plan.event_q.cpu()
    n_c = plan.content_order.numel()
    reread = ((ew == n_c) & (eq < n_c)).tolist()
    runs, cur = [], []
    for e, flag in enumerate(reread):
        if flag:
            cur.append(int(eq[e]))
        elif cur:
            runs.append(cur)
            cur = []
    if cur:
        runs.append(cur)
    rows = next(r for r in runs if len(r) == size)
    return plan.content_order.cpu()[torch.tensor(rows)]


@pytest.mark.parametrize("seed", range(4))
def test_layer_core_shared_hidden_rows(gdn, seed):
    """A two-branch plan built like ops/gated_delta_layout.py:66-83 (Bi_I+CQ_T): the generation
    branch re-writes the prefix's hidden rows as its own content rows, so content_order repeats
    rows; the projection gradient of such a row is the sum over its content rows."""
    import layer_harness as layer

    H = 16
    plan = layer.two_branch_plan(260, 70, prefix=40, suffix=50, image_groups=(30,), seed=9)
    order = plan.content_order
    assert torch.unique(order).numel() < order.numel()
    print(f"case layer core, shared hidden rows: {plan.hidden_length} rows, {order.numel()} content, seed {seed}",
          flush=True)
    gen = torch.Generator().manual_seed(91 + 1000 * seed)
    proj = (torch.randn(plan.hidden_length, 4 * H * 128 + 2 * H, generator=gen) * 0.7).bfloat16()
    compare_layer(*layer_parity(plan, proj, H, gen), H)


@pytest.mark.parametrize("seed", range(4))
def test_layer_core_h32_and_column_sliced_projection(gdn, seed):
    """H = 32 through the fused layer, with the projection a column slice of a wider tensor (its row
    stride is larger than its width): results equal the contiguous projection's."""
    from cqgdn import events
    import layer_harness as layer

    H, S = 32, 4096
    P = 4 * S + 2 * H
    plan = layer.cq_layer_plan(160, 40, image_groups=(20,), seed=10)
    print(f"case layer core H=32: {plan.hidden_length} rows, seed {seed}", flush=True)
    gen = torch.Generator().manual_seed(101 + 1000 * seed)
    proj = (torch.randn(plan.hidden_length, P, generator=gen) * 0.7).bfloat16()
    compare_layer(*layer_parity(plan, proj, H, gen), H)
    if seed:
        return
    # the same projection inside a wider tensor (row stride P + 72), against the contiguous one
    params = _layer_params(H, gen)
    wide = torch.zeros(plan.hidden_length, P + 72, dtype=torch.bfloat16)
    wide[:, 24:24 + P] = proj
    dout = (torch.randn(plan.hidden_length, S, generator=gen) * 0.1).bfloat16().to(DEV)
    res = []
    for src in (proj.to(DEV), wide.to(DEV)):
        src = src.detach().requires_grad_()
        p = src if src.shape[1] == P else src[:, 24:24 + P]
        out = events.layer_core(p, *params, plan, heads=H)
        out.backward(dout)
        g = src.grad if src.shape[1] == P else src.grad[:, 24:24 + P]
        res.append((out.detach(), g))
    torch.cuda.synchronize()
    assert torch.equal(res[0][0], res[1][0])
    assert torch.equal(res[0][1], res[1][1])


def test_layer_decode_step_h32(gdn):
    """The layer's decode step at H = 32 against the float64 oracle step, two steps, N = 2."""
    from cqgdn import events

    N, H, K = 2, 32, 4
    S, P = H * 128, 4 * H * 128 + 2 * H
    print("case layer decode H=32", flush=True)
    gen = torch.Generator().manual_seed(111)
    w = (torch.rand(3 * S, K, generator=gen) - 0.5).bfloat16()
    A_log = torch.rand(H, generator=gen).mul(3).add(0.01).log()
    dt_bias = torch.randn(H, generator=gen) * 0.5
    nw = 1 + 0.1 * torch.randn(128, generator=gen)
    hist = (torch.randn(N, K - 1, 3 * S, generator=gen) * 0.7).bfloat16()
    state = torch.randn(N, H, 128, 128, generator=gen) * 0.05
    cache = {"conv": hist.to(DEV), "state": state.to(DEV)}
    ref_hist, ref_state = hist.double(), state.double()
    dev = [t.to(DEV) for t in (w, A_log, dt_bias, nw)]
    for step in range(2):
        proj = (torch.randn(N, 2, P, generator=gen) * 0.7).bfloat16()
        out = events.layer_decode_step(proj.to(DEV), *dev, cache, heads=H)
        torch.cuda.synchronize()
        args = (proj[..., :3 * S], proj[..., 3 * S:4 * S].reshape(N, 2, H, 128), proj[..., 4 * S:4 * S + H],
                proj[..., 4 * S + H:], w, A_log, dt_bias, nw)
        ref_out, ref_hist, ref_state = O.layer_decode_step(*args, ref_hist, ref_state)
        assert_close_bf16(f"out step {step}", out.cpu(), ref_out.reshape(N, 2, S))
        assert torch.equal(cache["conv"].cpu().double(), ref_hist)
        assert_close_bf16(f"state step {step}", cache["state"].cpu(), ref_state)


def test_whole_layer_at_benchmark_plan_matches_float64_recurrence(gdn):
    """The layer at the first row of the reference's layer benchmark (scripts/benchmark_gdn.py:34-64):
    width 2048, content 2048 with 1675 CQ queries and two image groups -- the 4221-event image-CQ plan
    bench.py times -- in bf16 on the GPU, three ways:

    * ``oracle``: the reference's torch code around the float64 chunked oracle recurrence (on the CPU);
    * ``hip``: the same torch code around this backend's ``delta`` (the reference's provider-against-
      provider comparison, one glue, two recurrences);
    * ``fused``: everything between the projections in the fused kernels (``events.layer_core``).

    y, dx and the input-projection gradient dw of ``hip`` and ``fused`` against ``oracle`` within 2e-2,
    with the reference benchmark's relative RMS (rms(a - b) / rms(b), b the oracle path) printed for each."""
    import layer_harness as layer

    print("case whole layer at the benchmark plan: content 2048, 1675 queries, 4221 events", flush=True)
    torch.manual_seed(872)
    model = layer.GatedDeltaLayer().to(DEV, torch.bfloat16)
    model.A_log.data = model.A_log.data.float()
    model.norm_weight.data = model.norm_weight.data.float()
    plan = layer.cq_layer_plan(2048, 1675).to(DEV)
    assert len(plan.event_q) == 4221
    gen = torch.Generator().manual_seed(873)
    x = torch.randn(plan.hidden_length, 1, 2048, generator=gen).bfloat16().to(DEV)
    up = (torch.randn(plan.hidden_length, 1, 2048, generator=gen) / 100).bfloat16().to(DEV)

    def run(recurrence, fused):
        model.zero_grad(set_to_none=True)
        xx = x.clone().requires_grad_()
        y = model(xx, plan, recurrence=recurrence, fused=fused)
        (y * up).sum().backward()
        torch.cuda.synchronize()
        return y.detach().float().cpu(), xx.grad.float().cpu(), model.in_proj_all.weight.grad.float().cpu()

    def oracle(q, k, v, g, b, p):
        ins = [t.detach().double().cpu().requires_grad_() for t in (q, k, v, g, b)]
        out = O.chunk_delta(*ins, p.event_bounds, normalize=True)

        class Bridge(torch.autograd.Function):  # float64 CPU recurrence inside the bf16 GPU graph
            @staticmethod
            def forward(ctx, *dev_ins):
                return out.detach().to(q.device, q.dtype)

            @staticmethod
            def backward(ctx, dy):
                grads = torch.autograd.grad(out, ins, dy.double().cpu())
                return tuple(gr.to(t.device, t.dtype) for gr, t in zip(grads, (q, k, v, g, b)))

        return Bridge.apply(q, k, v, g, b)

    want = run(oracle, False)
    for label, got in (("hip", run(None, False)), ("fused", run(None, True))):
        rms = {n: float((b.double() - a.double()).square().mean().sqrt() / b.double().square().mean().sqrt())
               for n, a, b in zip(("y", "dx", "dw"), got, want)}
        print(f"  {label} vs oracle, relative RMS: y={rms['y']:.2e} dx={rms['dx']:.2e} dw={rms['dw']:.2e}", flush=True)
        for name, a, b in zip(("y", "dx", "dW_in"), got, want):
            assert_close_bf16(f"{label} {name}", a, b.double())


def test_decode_steps_replay_in_a_hip_graph(gdn):
    """The decode loop of config 4's shape captured once in a HIP graph (as a serving loop runs it):
    every replay -- with eager work and synchronizations of the program between them -- gives exactly
    the states and outputs of the same steps run eagerly from the same starting states."""
    N, H, E, steps = 16, 16, 2, 6
    print(f"case decode graph: N={N} H={H} E={E} steps={steps}", flush=True)
    gen = torch.Generator().manual_seed(44)
    q = O.l2norm(torch.randn(N, E, H, 128, generator=gen)).bfloat16().to(DEV)
    k = O.l2norm(torch.randn(N, E, H, 128, generator=gen)).bfloat16().to(DEV)
    v = torch.randn(N, E, H, 128, generator=gen).bfloat16().to(DEV)
    g = (-torch.nn.functional.softplus(torch.randn(N, E, H, generator=gen))).to(DEV)
    b = torch.randn(N, E, H, generator=gen).sigmoid().to(DEV)
    init = [(torch.randn(N, H, 128, 128, generator=gen) * 0.02).to(DEV) for _ in range(2)]
    outs = [torch.empty(N, E, H, 128, dtype=torch.bfloat16, device=DEV) for _ in range(steps)]

    def run(states):
        for i in range(steps):
            gdn.recurrent(q, k, v, g, b, states[i % 2], outs[i])

    eager_states = [s.clone() for s in init]
    run(eager_states)
    torch.cuda.synchronize()
    eager_outs = [o.clone() for o in outs]
    states = [s.clone() for s in init]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run([s.clone() for s in init])  # warm-up off the capture
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run(states)
    for replay in range(3):
        for s, s0 in zip(states, init):
            s.copy_(s0)
        for o in outs:
            o.fill_(0)
        _ = (torch.randn(256, 256, device=DEV) @ torch.randn(256, 256, device=DEV)).sum().item()  # eager work between
        graph.replay()
        torch.cuda.synchronize()
        for s, e in zip(states, eager_states):
            assert torch.equal(s, e), f"replay {replay}: state differs"
        for o, e in zip(outs, eager_outs):
            assert torch.equal(o, e), f"replay {replay}: output differs"


def test_fused_mode_matches_cached_mode(gdn, monkeypatch):
    """DELTA_HIP_MODE=fused keeps only the inputs between the forward and the backward and rebuilds
    the workspace in the backward (the reference's default mode, ops/gated_delta_net.py:143-156,192-194):
    output and every gradient equal the cached mode's exactly (same kernels on the same inputs)."""
    bounds = (0, 130, 300)
    print(f"case fused vs cached mode, bounds={bounds}", flush=True)
    xs = inputs(300, 16, seed=88)
    do = torch.randn(1, 300, 16, 128, generator=torch.Generator().manual_seed(89)).bfloat16()
    res = {}
    for mode in ("cached", "fused"):
        monkeypatch.setattr(gdn, "MODE", mode)
        res[mode] = fwd_bwd(gdn, xs, bounds, do)
    (y_c, g_c), (y_f, g_f) = res["cached"], res["fused"]
    assert torch.equal(y_c, y_f)
    for a, b in zip(g_c, g_f):
        assert torch.equal(a, b)
    check_against_oracle(xs, bounds, do, y_f, g_f)


def test_fused_mode_matches_cached_mode_at_config2_size(gdn, monkeypatch):
    """At config 2's size (T = 9216, H = 16) the fused backward's rebuilt state scan runs beside its
    local kernel and reverse scan for about 100 us; the last kernel must see its h and v_new, so every
    gradient equals the cached mode's bitwise (the cached mode is checked against the oracle at this
    size in test_gpu_parity.py)."""
    from cqgdn import synthetic

    T, mask, bounds = synthetic.config_events(2, seed=0)
    print(f"case fused vs cached mode, config 2 T={T}", flush=True)
    xs = inputs(T, 16, seed=2, readonly=mask)
    do = torch.randn(1, T, 16, 128, generator=torch.Generator().manual_seed(102)).bfloat16()
    res = {}
    for mode in ("cached", "fused"):
        monkeypatch.setattr(gdn, "MODE", mode)
        res[mode] = fwd_bwd(gdn, xs, bounds, do)
    (y_c, g_c), (y_f, g_f) = res["cached"], res["fused"]
    assert torch.equal(y_c, y_f)
    for name, a, b in zip(("dq", "dk", "dv", "dg", "dbeta"), g_c, g_f):
        assert torch.equal(a, b), name


@pytest.mark.parametrize("T,bounds,H,dtype", [(700, (0, 300, 700), 8, torch.bfloat16),
                                               (4200, (0, 4200), 16, torch.bfloat16),
                                               (4200, (0, 4200), 16, torch.float16)])
def test_bwd_recompute_graph_replay(gdn, T, bounds, H, dtype):
    """cqgdn_bwd_recompute (the fused-mode backward: forward rebuilt in the call, its state scan on a
    second stream joined back by events) captured in a HIP graph, at two sizes and with fp16 inputs
    (whose range scales are formed inside the call): each replay, with eager work between, equals the
    eager call bitwise."""
    print(f"case bwd_recompute graph replay T={T} bounds={bounds} H={H} {dtype}", flush=True)
    q, k, v, g, b = (x.to(DEV).contiguous() for x in inputs(T, H, seed=4242))
    q, k, v = (x.to(dtype) for x in (q, k, v))
    dy = torch.randn(1, T, H, 128, generator=torch.Generator().manual_seed(4243)).to(dtype).to(DEV)

    def run():
        return gdn._backward(q, k, v, g, b, None, dy, bounds, True, 128 ** -0.5)

    eager = [x.clone() for x in run()]
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run()  # warm-up off the capture
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = run()
    for replay in range(3):
        for o in outs:
            o.fill_(0)
        _ = (torch.randn(256, 256, device=DEV) @ torch.randn(256, 256, device=DEV)).sum().item()  # eager work between
        graph.replay()
        torch.cuda.synchronize()
        for name, o, e in zip(("dq", "dk", "dv", "dg", "dbeta"), outs, eager):
            assert torch.equal(o, e), f"replay {replay}: {name} differs"


def _bwd_direct(gdn, xs, bounds, do, beside, monkeypatch):
    """cqgdn_bwd through the C ABI with its workspace in hand; beside=False sets CQGDN_DKW_BESIDE_SCAN=0."""
    from cqgdn import _lib

    monkeypatch.setenv("CQGDN_DKW_BESIDE_SCAN", "1" if beside else "0")
    T, H = xs[0].shape[1], xs[0].shape[2]
    q, k, v, g, b = (x.to(DEV).contiguous() for x in xs)
    do_dev = do.to(DEV)
    _, _, ws = gdn._forward(q, k, v, g, b, bounds, True, 128 ** -0.5, training=True)
    _, table, doc = gdn.device_metadata(bounds, DEV)
    nc = table.shape[0]
    bws = torch.full((_lib.lib().cqgdn_bwd_workspace_size(T, H, nc),), 0x5A, dtype=torch.uint8, device=DEV)
    dq, dk, dv = (torch.empty_like(v) for _ in range(3))
    dg, db = torch.empty_like(g), torch.empty_like(b)
    P = gdn._ptr
    flags = _lib.NORMALIZE | _lib.TRAINING | (_lib.FP16 if q.dtype == torch.float16 else 0)
    gdn.call("cqgdn_bwd", P(q), P(k), P(v), P(g), P(b), P(do_dev), T, H, P(table), nc, P(doc), len(bounds) - 1,
             128 ** -0.5, flags, P(ws), ws.numel(), P(bws), bws.numel(), P(dq), P(dk), P(dv), P(dg), P(db),
             gdn._stream(q.device))
    torch.cuda.synchronize()
    sync = view(bws, _lib.bwd_offsets(T, H, nc)["sync"], torch.int32, (nc * H + 1,)).cpu()
    return [x.cpu() for x in (dq, dk, dv, dg, db)], sync[:-1].view(nc, H), int(sync[-1])


def _beside(H, n_docs, nc):
    """Whether the library runs the kernel after a state scan beside it: every scan workgroup (one per
    head, 16-wide value slice and document, a whole CU each) is resident at once on at most half of the
    CUs, and documents average at least 64 chunks."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    return H * 8 * n_docs * 2 <= cus and nc >= 64 * n_docs


@pytest.mark.parametrize("kind", ["config2", "two_long_docs_h4", "two_long_docs_h4_fp16", "three_docs"])
def test_bwd_dkw_beside_scan_matches_after_scan(gdn, kind, monkeypatch):
    """cqgdn_bwd runs bwd_dkw on a second stream beside the reverse scan, taking chunks in the order
    the scan finishes them, when every scan workgroup is resident at once and the documents are long:
    each chunk-head waits, bounded, until all eight value slices have announced its dS and dVn
    (device-scope stores, then an atomic count).  Otherwise, and
    with CQGDN_DKW_BESIDE_SCAN=0, bwd_dkw runs after the scan.  Both orders give bit-identical
    gradients.  The workspace's counts show which path ran: beside the scan every chunk-head's count
    ends at 8 and the resident count at the scan's workgroup count; after it both stay at bwd_local's
    zeros.  The fp16 case runs the fp16 kernels (CQGDN_FP16) on fp16 inputs."""
    from cqgdn import synthetic

    H = 4 if "h4" in kind else 16
    if kind == "config2":
        T, mask, bounds = synthetic.config_events(2, seed=0)
        xs = inputs(T, H, seed=21, readonly=mask)
    elif kind.startswith("two_long_docs_h4"):
        T, bounds = 8400, (0, 4200, 8400)
        xs = inputs(T, H, seed=22)
    else:
        T, bounds = 1200, (0, 300, 777, 1200)
        xs = inputs(T, H, seed=23)
    n_docs = len(bounds) - 1
    fits = _beside(H, n_docs, gdn.device_metadata(bounds, DEV)[1].shape[0])
    print(f"case bwd_dkw beside the reverse scan ({kind}): T={T} docs={n_docs} fits={fits}", flush=True)
    do = torch.randn(1, T, H, 128, generator=torch.Generator().manual_seed(24)).bfloat16()
    if kind.endswith("fp16"):
        xs = [x.half() if x.dim() == 4 else x for x in xs]
        do = do.half()
    after, ready_a, resident_a = _bwd_direct(gdn, xs, bounds, do, False, monkeypatch)
    beside, ready_b, resident_b = _bwd_direct(gdn, xs, bounds, do, True, monkeypatch)
    for name, a, b in zip(("dq", "dk", "dv", "dg", "dbeta"), after, beside):
        assert not torch.isnan(a.float()).any(), name
        assert torch.equal(a, b), name
    assert not ready_a.any() and resident_a == 0
    assert (kind != "three_docs") == fits
    assert all(x.dtype == xs[0].dtype for x in beside[:3])
    if fits:
        assert bool((ready_b == 8).all()) and resident_b == H * 8 * n_docs, (ready_b.unique(), resident_b)
    else:
        assert not ready_b.any() and resident_b == 0
    if kind.startswith("two_long_docs_h4"):  # two documents, four heads
        ref = O.chunk_delta_backward(*(x.double() for x in xs), do.double(), bounds)
        for name, x, r in zip(("dq", "dk", "dv", "dg", "dbeta"), beside, ref):
            assert_close_bf16(name, x, r, tol=TOL_FP16 if kind.endswith("fp16") else TOL_BF16)


# seeds chosen to cover 4 heads x 3 and 4 documents, 8 x 1 and 2, 16 x 1, in both types
@pytest.mark.parametrize("seed", [300, 302, 306, 308, 310, 314, 316, 318])
def test_bwd_dkw_beside_scan_random_cases_bit_identical(gdn, seed, monkeypatch):
    """Random cases that run bwd_dkw beside the reverse scan: 4, 8 or 16 heads, as many documents
    (at most four) as leave half of the CUs free, each of 64 to 93 chunks with a ragged end, a fifth
    of the rows read-only at random, bf16 or fp16.  The gradients equal those of the after-the-scan
    path bitwise, none is NaN, and every chunk-head's count reaches the scan's eight value slices."""
    rng = np.random.default_rng(seed)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    H = int(rng.choice([4, 8, 16]))
    n_docs = int(rng.integers(1, max(1, min(4, cus // (16 * H))) + 1))
    lens = [int(rng.integers(64 * 64, 64 * 94)) for _ in range(n_docs)]
    bounds = tuple(int(x) for x in np.concatenate([[0], np.cumsum(lens)]))
    T = bounds[-1]
    fp16 = bool(rng.integers(0, 2))
    mask = torch.from_numpy(rng.random(T) < 0.2)
    nc = gdn.device_metadata(bounds, DEV)[1].shape[0]
    print(f"case random beside seed={seed}: H={H} docs={n_docs} T={T} chunks={nc} fp16={fp16}", flush=True)
    assert _beside(H, n_docs, nc)
    xs = inputs(T, H, seed=seed, readonly=mask)
    do = torch.randn(1, T, H, 128, generator=torch.Generator().manual_seed(seed + 1)).bfloat16()
    if fp16:
        xs = [x.half() if x.dim() == 4 else x for x in xs]
        do = do.half()
    after, ready_a, resident_a = _bwd_direct(gdn, xs, bounds, do, False, monkeypatch)
    beside, ready_b, resident_b = _bwd_direct(gdn, xs, bounds, do, True, monkeypatch)
    for name, a, b in zip(("dq", "dk", "dv", "dg", "dbeta"), after, beside):
        assert not torch.isnan(a.float()).any(), name
        assert torch.equal(a, b), name
    assert not ready_a.any() and resident_a == 0
    assert bool((ready_b == 8).all()) and resident_b == H * 8 * n_docs, (ready_b.unique(), resident_b)


def test_bwd_dkw_wait_gives_up_with_nan_not_a_hang(gdn, monkeypatch):
    """bwd_dkw's wait for a chunk of the reverse scan is bounded.  CQGDN_TEST_DKW_GIVE_UP=1 (failure
    tests only) makes every chunk wait for a count the scan never reaches, four polls long: the call
    still ends, the gradients that depend on the scan's dS and dV_new (dk, dv, dg, dbeta) are NaN in
    every element, and dq, which does not, equals the normal call's bitwise."""
    from cqgdn import synthetic

    H = 16
    T, mask, bounds = synthetic.config_events(2, seed=0)
    print(f"case bwd_dkw wait give-up, config 2 T={T}", flush=True)
    xs = inputs(T, H, seed=25, readonly=mask)
    do = torch.randn(1, T, H, 128, generator=torch.Generator().manual_seed(26)).bfloat16()
    good, _, _ = _bwd_direct(gdn, xs, bounds, do, True, monkeypatch)
    monkeypatch.setenv("CQGDN_TEST_DKW_GIVE_UP", "1")
    bad, ready, resident = _bwd_direct(gdn, xs, bounds, do, True, monkeypatch)
    assert bool((ready == 8).all()) and resident == H * 8  # the scan itself ran and announced every chunk
    assert torch.equal(bad[0], good[0]), "dq"
    for name, x in zip(("dk", "dv", "dg", "dbeta"), bad[1:]):
        assert bool(torch.isnan(x.float()).all()), name


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_bwd_beside_scan_graph_replay(gdn, dtype):
    """The cached backward with bwd_dkw beside the reverse scan (second stream, fork and join events,
    the counts zeroed by bwd_local inside the call; with fp16 inputs also the scale of dO) captured in a
    HIP graph: each replay, with eager work between, equals the eager call bitwise."""
    T, bounds, H = 4200, (0, 4200), 16
    print(f"case cached bwd beside the scan, graph replay T={T} H={H} {dtype}", flush=True)
    q, k, v, g, b = (x.to(DEV).contiguous() for x in inputs(T, H, seed=4343))
    q, k, v = (x.to(dtype) for x in (q, k, v))
    dy = torch.randn(1, T, H, 128, generator=torch.Generator().manual_seed(4344)).to(dtype).to(DEV)
    _, _, ws = gdn._forward(q, k, v, g, b, bounds, True, 128 ** -0.5, training=True)

    def run():
        return gdn._backward(q, k, v, g, b, ws, dy, bounds, True, 128 ** -0.5)

    eager = [x.clone() for x in run()]
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run()  # warm-up off the capture
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = run()
    for replay in range(4):
        for o in outs:
            o.fill_(0)
        _ = (torch.randn(256, 256, device=DEV) @ torch.randn(256, 256, device=DEV)).sum().item()  # eager work between
        graph.replay()
        torch.cuda.synchronize()
        for name, o, e in zip(("dq", "dk", "dv", "dg", "dbeta"), outs, eager):
            assert torch.equal(o, e), f"replay {replay}: {name} differs"


@pytest.mark.parametrize("mode", ["cached", "fused"])
def test_delta_fp16_inputs_match_oracle(gdn, monkeypatch, mode):
    """fp16 q/k/v, which the reference's delta accepts (ops/gated_delta_net.py:233-234), run the fp16
    kernels (CQGDN_FP16) forward and backward: output and gradients come back in the input dtypes and
    match the float64 oracle of the same fp16 values to TOL_FP16.  The values are drawn in fp32 and
    rounded to fp16, so most of them are not bf16 values.  Beside it, the same values rounded to bf16
    run through the bf16 kernels (8-bit mantissas in place of fp16's 11), measured against the same
    oracle: every output of the fp16 route is at least four times closer."""
    monkeypatch.setattr(gdn, "MODE", mode)
    T, bounds, H = 257, (0, 100, 257), 8
    print(f"case fp16 inputs T={T} bounds={bounds} mode={mode}", flush=True)
    gen = torch.Generator().manual_seed(1616)
    _, _, _, g, b = inputs(T, H, seed=1616)
    q, k, v = (torch.randn(1, T, H, 128, generator=gen).half() for _ in range(3))
    assert not torch.equal(q.bfloat16().half(), q)  # genuinely fp16 values
    do = torch.randn(1, T, H, 128, generator=torch.Generator().manual_seed(17)).half()
    y, grads = fwd_bwd(gdn, [q, k, v, g, b], bounds, do)
    assert y.dtype == torch.float16 and [x.dtype for x in grads] == [torch.float16] * 3 + [torch.float32] * 2
    yb, gradsb = fwd_bwd(gdn, [q.bfloat16(), k.bfloat16(), v.bfloat16(), g, b], bounds, do.bfloat16())
    xs = [x.double() for x in (q, k, v, g, b)]
    ref = [O.chunk_delta(*xs, bounds)] + list(O.chunk_delta_backward(*xs, do.double(), bounds))
    for name, x, xb, r in zip(("o", "dq", "dk", "dv", "dg", "dbeta"), [y] + grads, [yb] + gradsb, ref):
        assert_close_bf16(name, x, r, tol=TOL_FP16)
        e16, eb = rel_l2(x, r), rel_l2(xb, r)
        print(f"    bf16 route: rel_l2={eb:.3e} ({eb / e16:.1f}x the fp16 route's)", flush=True)
        assert e16 * 4 <= eb, (name, e16, eb)


@pytest.mark.parametrize("kind", ["random", "aligned"])
def test_delta_fp16_range_scales(gdn, kind):
    """The fp16 route's power-of-two scales at large magnitudes.  One document of 8192 events with no
    decay (g = 0: the state gradient sums over the whole document), v up to ~340 and dO up to ~1400:
    without the scales, the products dP = dO v^T (~1e5) would leave fp16's range (65504).  "random"
    matches the float64 oracle of the same fp16 values to TOL_FP16, every value finite.

    "aligned" makes every event push the same way (q and k near one direction, v and dO positive):
    the states then follow v so closely that v_new = v - S k cancels, an ill-conditioned input on
    which any finite-precision route loses digits (on MI355X the bf16 route measured up to 1e-1
    against the oracle of its own bf16 inputs).  There every output of the fp16 route must be at
    least four times closer to its oracle than the bf16 route is to its own, and finite."""
    T, H = 8192, 4
    bounds = (0, T)
    _, _, _, _, b = inputs(T, H, seed=1818)
    gen = torch.Generator().manual_seed(1819)
    q, k = (torch.randn(1, T, H, 128, generator=gen) for _ in range(2))
    v = torch.randn(1, T, H, 128, generator=gen) * 64
    do = torch.randn(1, T, H, 128, generator=gen) * 256
    if kind == "aligned":
        q, k = q * 0.1 + 1, k * 0.1 + 1
        v, do = v.abs(), do.abs()
    g = torch.zeros(1, T, H)
    q, k, v, do = (x.half() for x in (q, k, v, do))
    print(f"case fp16 range ({kind}) T={T} H={H} no decay: max|v|={float(v.float().abs().max()):.3g} "
          f"max|dO|={float(do.float().abs().max()):.3g}", flush=True)
    y, grads = fwd_bwd(gdn, [q, k, v, g, b], bounds, do)
    xs = [x.double() for x in (q, k, v, g, b)]
    ref = [O.chunk_delta(*xs, bounds)] + list(O.chunk_delta_backward(*xs, do.double(), bounds))
    names = ("o", "dq", "dk", "dv", "dg", "dbeta")
    if kind == "random":
        for name, x, r in zip(names, [y] + grads, ref):
            print(f"    max|{name}| = {float(r.abs().max()):.3g}", flush=True)
            assert_close_bf16(name, x, r, tol=TOL_FP16)
        return
    qb, kb, vb, dob = (x.bfloat16() for x in (q, k, v, do))
    yb, gradsb = fwd_bwd(gdn, [qb, kb, vb, g, b], bounds, dob)
    xsb = [x.double() for x in (qb, kb, vb, g, b)]
    refb = [O.chunk_delta(*xsb, bounds)] + list(O.chunk_delta_backward(*xsb, dob.double(), bounds))
    for name, x, r, xb, rb in zip(names, [y] + grads, ref, [yb] + gradsb, refb):
        assert torch.isfinite(x.float()).all(), name
        e16, eb = rel_l2(x, r), rel_l2(xb, rb)
        print(f"  {name}: fp16 route rel_l2={e16:.3e}, bf16 route rel_l2={eb:.3e} ({eb / e16:.1f}x)", flush=True)
        assert e16 * 4 <= eb, (name, e16, eb)


def test_prefill_and_recurrent_fp16_inputs_match_oracle(gdn):
    """fp16 q/k/v through the inference entry points as through delta: prefill returns its output
    in fp16 with fp32 states, and recurrent writes its fp16 output in place; both match the
    float64 oracle of the same fp16 values (outputs to 2e-2, states to 1e-3)."""
    T, bounds, H = 300, (0, 120, 300), 8
    print(f"case fp16 prefill T={T} bounds={bounds} then 3 decode steps", flush=True)
    q, k, v, g, b = inputs(T, H, seed=1717)
    q, k, v = (x.float().half() for x in (q, k, v))
    o, state = gdn.prefill(*(x.to(DEV) for x in (q, k, v, g, b)), bounds)
    torch.cuda.synchronize()
    assert o.dtype == torch.float16 and state.dtype == torch.float32
    ref, ref_state = O.chunk_delta(*(x.double() for x in (q, k, v, g, b)), bounds, output_final_state=True)
    assert_close_bf16("o", o.cpu(), ref)
    assert rel_l2(state, ref_state) <= TOL_STATE
    # decode both documents three steps from their prefill states (value-first)
    gen = torch.Generator().manual_seed(1718)
    st = state.transpose(-1, -2).contiguous()
    ref_st = ref_state.transpose(-1, -2).contiguous()
    for step in range(3):
        qs = O.l2norm(torch.randn(2, 1, H, 128, generator=gen)).half()
        ks = O.l2norm(torch.randn(2, 1, H, 128, generator=gen)).half()
        vs = torch.randn(2, 1, H, 128, generator=gen).half()
        gs = -torch.nn.functional.softplus(torch.randn(2, 1, H, generator=gen))
        bs = torch.randn(2, 1, H, generator=gen).sigmoid()
        out = torch.empty(2, 1, H, 128, dtype=torch.float16, device=DEV)
        gdn.recurrent(*(x.to(DEV) for x in (qs, ks, vs, gs, bs)), st, out)
        expected = O.decode_step(qs.double(), ks.double(), vs.double(), gs.double(), bs.double(), ref_st)
        torch.cuda.synchronize()
        assert_close_bf16(f"decode o step {step}", out.cpu(), expected)
        assert rel_l2(st, ref_st) <= TOL_STATE


# ---- fewer key heads than value heads (models/backbone_qwen35.py:182-183, models/decoding.py:52-53)

@pytest.mark.parametrize("seed", range(4))
@pytest.mark.parametrize("H,HK,kind", [(32, 16, "image-CQ"), (16, 4, "two-branch")])
def test_layer_core_fewer_key_heads(gdn, H, HK, kind, seed):
    """layer_core with H value heads and HK < H key heads (the Qwen3.5-9B shape per rank is 32 and
    16) against the reference's layer code in float64, which repeat_interleaves q, k and the query
    conv output: the output, every projection-gradient column block (the q and k blocks sum their
    value heads' gradients) and the parameter gradients.  The two-branch plan repeats hidden rows."""
    import layer_harness as layer

    if kind == "image-CQ":
        plan = layer.cq_layer_plan(200, 50, image_groups=(24,), seed=12)
    else:
        plan = layer.two_branch_plan(220, 60, prefix=30, suffix=40, image_groups=(20,), seed=13)
    print(f"case layer core H={H} key heads={HK} ({kind}): {plan.hidden_length} rows, seed {seed}", flush=True)
    gen = torch.Generator().manual_seed(121 + H + 1000 * seed)
    P = (2 * HK + 2 * H) * 128 + 2 * H
    proj = (torch.randn(plan.hidden_length, P, generator=gen) * 0.7).bfloat16()
    compare_layer(*layer_parity(plan, proj, H, gen, HK), H, HK)


def _gqa_decode_params(H, HK, K, gen):
    C = (2 * HK + H) * 128
    w = (torch.rand(C, K, generator=gen) - 0.5).bfloat16()
    A_log = torch.rand(H, generator=gen).mul(3).add(0.01).log()
    dt_bias = torch.randn(H, generator=gen) * 0.5
    nw = 1 + 0.1 * torch.randn(128, generator=gen)
    return w, A_log, dt_bias, nw


def test_layer_decode_step_fewer_key_heads(gdn):
    """The layer's decode step with 32 value heads and 16 key heads against the float64 oracle step,
    three steps, N = 3: outputs, the value-first state, and the conv history bit-exact (its key
    channels are shifted by the second launch, after every workgroup of the step has read them)."""
    from cqgdn import events

    N, H, HK, K = 3, 32, 16, 4
    S, C = H * 128, (2 * HK + H) * 128
    P = C + S + 2 * H
    print(f"case layer decode H={H} key heads={HK}", flush=True)
    gen = torch.Generator().manual_seed(131)
    w, A_log, dt_bias, nw = _gqa_decode_params(H, HK, K, gen)
    hist = (torch.randn(N, K - 1, C, generator=gen) * 0.7).bfloat16()
    state = torch.randn(N, H, 128, 128, generator=gen) * 0.05
    cache = {"conv": hist.to(DEV), "state": state.to(DEV)}
    ref_hist, ref_state = hist.double(), state.double()
    dev = [t.to(DEV) for t in (w, A_log, dt_bias, nw)]
    for step in range(3):
        proj = (torch.randn(N, 2, P, generator=gen) * 0.7).bfloat16()
        out = events.layer_decode_step(proj.to(DEV), *dev, cache, heads=H, key_heads=HK)
        torch.cuda.synchronize()
        args = (proj[..., :C], proj[..., C:C + S].reshape(N, 2, H, 128), proj[..., C + S:C + S + H],
                proj[..., C + S + H:], w, A_log, dt_bias, nw)
        ref_out, ref_hist, ref_state = O.layer_decode_step(*args, ref_hist, ref_state)
        assert_close_bf16(f"out step {step}", out.cpu(), ref_out.reshape(N, 2, S))
        assert torch.equal(cache["conv"].cpu().double(), ref_hist), "conv history differs"
        assert_close_bf16(f"state step {step}", cache["state"].cpu(), ref_state)


def test_layer_prefill_then_decode_fewer_key_heads(gdn):
    """Prefill with the uncommitted target and one decode step equal the one-shot prefill of the
    extended plan, with 16 value heads and 8 key heads."""
    from cqgdn import events
    from gdn_testlib import decode_plans

    n, H, HK, K = 150, 16, 8, 4
    S, C = H * 128, (2 * HK + H) * 128
    P = C + S + 2 * H
    print(f"case prefill -> decode H={H} key heads={HK}", flush=True)
    gen = torch.Generator().manual_seed(141)
    w, A_log, dt_bias, nw = (t.to(DEV) for t in _gqa_decode_params(H, HK, K, gen))
    pre_plan, one_plan = decode_plans(n, K)
    proj = (torch.randn(n + 2, P, generator=gen) * 0.7).bfloat16().to(DEV)
    kw = dict(heads=H, key_heads=HK)
    _, cache = events.layer_prefill(proj[:n + 1], w, A_log, dt_bias, nw, pre_plan, **kw)
    assert torch.equal(cache["conv"][0], proj[n - K + 1:n, :C])
    out = events.layer_decode_step(proj[n:n + 2], w, A_log, dt_bias, nw, cache, **kw)
    one, one_cache = events.layer_prefill(proj, w, A_log, dt_bias, nw, one_plan, **kw)
    torch.cuda.synchronize()
    assert_close_bf16("C and Q rows", out.cpu(), one[n:n + 2].double().cpu())
    assert_close_bf16("state", cache["state"].cpu(), one_cache["state"].double().cpu())
    assert torch.equal(cache["conv"][0], proj[n - K + 2:n + 1, :C])


def test_layer_decode_steps_replay_in_a_hip_graph(gdn):
    """Layer decode steps captured once in a HIP graph, with fewer key heads than value heads (so the
    capture holds the step kernel and the key-history shift): every replay -- with eager work and
    synchronizations between them -- gives exactly the outputs, conv history and states of the same
    steps run eagerly from the same starting cache."""
    from cqgdn import events

    N, H, HK, K, steps = 2, 16, 8, 4, 4
    S, C = H * 128, (2 * HK + H) * 128
    P = C + S + 2 * H
    print(f"case layer decode graph: N={N} H={H} key heads={HK} steps={steps}", flush=True)
    gen = torch.Generator().manual_seed(151)
    w, A_log, dt_bias, nw = (t.to(DEV) for t in _gqa_decode_params(H, HK, K, gen))
    projs = [(torch.randn(N, 2, P, generator=gen) * 0.7).bfloat16().to(DEV) for _ in range(steps)]
    hist0 = (torch.randn(N, K - 1, C, generator=gen) * 0.7).bfloat16().to(DEV)
    state0 = (torch.randn(N, H, 128, 128, generator=gen) * 0.05).to(DEV)
    kw = dict(heads=H, key_heads=HK)

    def run(cache):
        return [events.layer_decode_step(p, w, A_log, dt_bias, nw, cache, **kw) for p in projs]

    eager_cache = {"conv": hist0.clone(), "state": state0.clone()}
    eager_outs = [o.clone() for o in run(eager_cache)]
    torch.cuda.synchronize()
    cache = {"conv": hist0.clone(), "state": state0.clone()}
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run({"conv": hist0.clone(), "state": state0.clone()})  # warm-up off the capture
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = run(cache)
    for replay in range(3):
        cache["conv"].copy_(hist0)
        cache["state"].copy_(state0)
        _ = (torch.randn(256, 256, device=DEV) @ torch.randn(256, 256, device=DEV)).sum().item()  # eager work between
        graph.replay()
        torch.cuda.synchronize()
        for i, (o, e) in enumerate(zip(outs, eager_outs)):
            assert torch.equal(o, e), f"replay {replay}: output of step {i} differs"
        assert torch.equal(cache["conv"], eager_cache["conv"]), f"replay {replay}: conv history differs"
        assert torch.equal(cache["state"], eager_cache["state"]), f"replay {replay}: state differs"
