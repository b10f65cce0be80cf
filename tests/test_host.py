"""Host-side logic of the hip backend (no GPU): metadata helpers, argument checks, work model, bench CLI.

Mirrors the reference's host contract of ops/gated_delta_net.py: host_bounds
(:102-114), chunk_indices (:90-99), the argument checks of delta() (:217-249)
and the no-fallback rule (:1, :166-167).
"""

import subprocess
import sys
from pathlib import Path

import pytest
import torch

from cqgdn import gated_delta_net as gdn
from cqgdn import synthetic, workmodel
from oracle import gdn_oracle as O

ROOT = Path(__file__).resolve().parents[1]


def test_host_bounds_contract():
    assert gdn.host_bounds(None, None) is None
    cu = torch.tensor([0, 5, 9])
    assert gdn.host_bounds(cu, torch.tensor([0, 5, 9])) == (0, 5, 9)
    assert gdn.host_bounds(cu, [0, 5, 9]) == (0, 5, 9)
    with pytest.raises(ValueError, match="cu_seqlens_cpu"):
        gdn.host_bounds(cu, None)
    for bad in ([1, 5], [0, 5, 3], []):
        with pytest.raises(ValueError, match="Invalid packed sequence boundaries"):
            gdn.host_bounds(cu, bad)


def test_chunk_indices_pairs():
    assert gdn.chunk_indices(None, 64) is None
    assert gdn.chunk_indices((0, 3, 200), 64) == [0, 0, 1, 0, 1, 1, 1, 2, 1, 3]  # 197 events: 4 chunks
    assert gdn.chunk_indices((0, 0, 65), 64) == [1, 0, 1, 1]  # an empty document has no chunk


@pytest.mark.parametrize("bounds", [(0, 1), (0, 64), (0, 65), (0, 37, 129), (0, 0, 130, 130),
                                    synthetic.doc_bounds(32768, seed=6)])
def test_chunk_table_matches_oracle_spans(bounds):
    table, doc = gdn.chunk_table(bounds)
    spans = O.chunk_spans(bounds)
    assert [(int(a), int(a) + int(n)) for a, n in table.tolist()] == spans
    assert doc.tolist()[-1] == len(spans)
    for d, (a, b) in enumerate(zip(bounds, bounds[1:])):
        first, last = doc[d].item(), doc[d + 1].item()
        assert [s for s in spans if a <= s[0] < b] == spans[first:last]


def test_chunk_table_rejects_invalid_bounds():
    for bad in ((1, 5), (0, 5, 3)):
        with pytest.raises(ValueError):
            gdn.chunk_table(bad)


def _bf16(T=4, H=4):
    return [torch.zeros(1, T, H, 128, dtype=torch.bfloat16) for _ in range(3)] + \
        [torch.zeros(1, T, H), torch.zeros(1, T, H)]


def test_delta_argument_checks_match_reference():
    q, k, v, g, b = _bf16()
    with pytest.raises(NotImplementedError, match="zero initial state"):
        gdn.delta(q, k, v, g, b, initial_state=torch.zeros(1))
    with pytest.raises(NotImplementedError, match="zero initial state"):
        gdn.delta(q, k, v, g, b, output_final_state=True)
    with pytest.raises(ValueError, match="QKV must share"):
        gdn.delta(q.float(), k, v, g, b)
    with pytest.raises(ValueError, match="head dimension 128"):
        gdn.delta(q[..., :64], k[..., :64], v[..., :64], g, b)
    q5 = torch.zeros(1, 4, 5, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="supported local heads"):
        gdn.delta(q5, q5, q5, g[..., :1].expand(1, 4, 5), b[..., :1].expand(1, 4, 5))
    cu = torch.tensor([0, 3])
    with pytest.raises(ValueError, match="covering every token"):
        gdn.delta(q, k, v, g, b, cu_seqlens=cu, cu_seqlens_cpu=[0, 3])
    with pytest.raises(ValueError, match="QKV must share"):
        gdn.delta(q.half(), k, v, g, b)
    # fp16 q/k/v pass the checks (the reference accepts bf16 or fp16); on the CPU the GPU check rejects them
    with pytest.raises(ValueError, match="ROCm GPU"):
        gdn.delta(q.half(), k.half(), v.half(), g, b)


def test_mode_is_checked_like_the_reference(monkeypatch):
    """DELTA_HIP_MODE accepts the reference's two modes (ops/gated_delta_net.py:20,57-58)."""
    for mode in ("fused", "cached"):
        monkeypatch.setattr(gdn, "MODE", mode)
        gdn.initialize()
    monkeypatch.setattr(gdn, "MODE", "eager")
    with pytest.raises(ValueError, match="Unknown DELTA_HIP_MODE"):
        gdn.initialize()


def test_no_cpu_fallback():
    # the hip backend never computes on the CPU: CPU tensors are rejected, not silently handled
    with pytest.raises(ValueError, match="ROCm GPU"):
        gdn.delta(*_bf16())
    with pytest.raises(ValueError, match="ROCm GPU"):
        gdn.prefill(*_bf16(), (0, 4))
    q = torch.zeros(1, 4, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="ROCm GPU"):
        gdn.recurrent(q, q, q, torch.zeros(1, 4), torch.zeros(1, 4), torch.zeros(1, 4, 128, 128), q.clone())


def test_product_package_never_imports_the_oracle():
    pkg = ROOT / "cq-pretrain_amd"
    for path in pkg.rglob("*.py"):
        text = path.read_text()
        assert "oracle" not in text.replace("oracle/", ""), f"{path} references the oracle"


def test_workmodel_split_sums_to_algorithmic_totals():
    # forward 10 C^2 d + 6 C d^2 + (2/3) C^3 and backward 20 C^2 d + 12 C d^2 + 4 C^3 per (chunk, head)
    fwd = sum(workmodel.flops_per_chunk(k, 64) for k in workmodel.FWD_KERNELS)
    bwd = sum(workmodel.flops_per_chunk(k, 64) for k in workmodel.BWD_KERNELS)
    assert round(fwd) == 11_709_099
    assert bwd == 24_117_248
    # config 2: 2304 chunk-heads, 82.5 GFLOP fwd+bwd
    total = sum(workmodel.kernel_work(k, (0, 9216), 16)[0] for k in workmodel.FWD_KERNELS + workmodel.BWD_KERNELS)
    assert abs(total - 82.54e9) < 0.01e9
    # decode: 64 * 16 * 132,104 bytes per step
    assert workmodel.decode_bytes(64, 16) == 64 * 16 * 132_104


def test_synthetic_configs():
    T1, m1, b1 = synthetic.config_events(1)
    assert T1 == 2304 and m1[2048:].all() and not m1[:2048].any() and b1 == (0, 2304)
    T2, m2, b2 = synthetic.config_events(2)
    assert T2 == 9216 and int(m2.sum()) == 1024 and b2 == (0, 9216)
    T3, _, b3 = synthetic.config_events(3)
    assert b3[-1] == 32768 and all(256 <= b - a <= 4096 for a, b in zip(b3, b3[1:-1]))
    q, k, v, g, beta = synthetic.make_inputs(16, 2, 128, seed=0, readonly=torch.arange(16) >= 12)
    assert (k[:, 12:] == 0).all() and (v[:, 12:] == 0).all() and (g[:, 12:] == 0).all() and (beta[:, 12:] == 0).all()
    assert (g[:, :12] < 0).all() and ((beta[:, :12] > 0) & (beta[:, :12] < 1)).all()


def test_bench_refuses_more_than_one_gpu():
    proc = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                          timeout=120)
    assert proc.returncode == 2
    assert "one GPU" in proc.stderr


def test_layer_plan_structure():
    """Synthetic image-CQ plan: counts of the reference's benchmark rows, each content row written
    once in order, read-only events write the zero row, the query conv sees earlier content only,
    every hidden row takes one event's output."""
    import layer_harness as layer

    for content, queries, events in ((2048, 1675, 4221), (8192, 7819, 16509)):
        p = layer.cq_layer_plan(content, queries)
        assert len(p.event_q) == events and p.hidden_length == content + queries
        writes = p.event_write[p.event_write < content]
        assert torch.equal(writes, torch.arange(content))
        assert int((p.event_write == content).sum()) == events - content
        assert int((p.event_q >= content).sum()) == queries
        assert p.hidden_event.shape == (content + queries,) and int(p.hidden_event.max()) < events
        # a query event's conv history holds content written before it
        first_write = {int(c): e for e, c in enumerate(p.event_write.tolist()) if c < content}
        for j in range(0, queries, 97):
            e = int(p.hidden_event[content + j])
            for c in p.query_history[j].tolist():
                assert c == content or first_write[c] < e


def test_layer_forward_backward_on_cpu_with_oracle_recurrence():
    """The whole-layer mirror runs fwd+bwd on the CPU with the oracle as its recurrence."""
    import layer_harness as layer

    torch.manual_seed(0)
    model = layer.GatedDeltaLayer(width=64, heads=4).double()
    plan = layer.cq_layer_plan(40, 9, image_groups=(6, 5))
    x = torch.randn(plan.hidden_length, 1, 64, dtype=torch.float64, requires_grad=True)
    rec = lambda q, k, v, g, b, p: O.recurrent_delta(q, k, v, g, b, p.event_bounds, normalize=True)
    cv = lambda u, w, bounds: O.causal_conv1d(u, w, bounds)
    y = model(x, plan, recurrence=rec, conv=cv, norm=O.gated_rms_norm)
    assert y.shape == x.shape
    y.square().sum().backward()
    assert torch.isfinite(x.grad).all() and model.in_proj_all.weight.grad.abs().sum() > 0


def test_event_plan_inverse_maps_against_brute_force():
    """The host-built inverse maps of the fused layer kernels (q readers per content row, the
    writer of each content row, the reader of each query, the query-history entries per content
    row) against direct scans of the plan, on a packed two-document plan; bad plans raise."""
    from cqgdn import events
    import layer_harness as layer

    plan = layer.concat_plans(layer.cq_layer_plan(60, 17, image_groups=(9, 5), seed=1),
                              layer.cq_layer_plan(45, 11, image_groups=(7,), seed=2))
    ep = events.event_plan(plan, 4, "cpu")
    t = {k: v.long() for k, v in ep.tensors.items()}
    n_c, n_q = ep.n_content, ep.n_queries
    eq, ew, qh = plan.event_q.tolist(), plan.event_write.tolist(), plan.query_history.tolist()
    assert (ep.content_bounds, ep.covers_all) == ((0, 60, 105), True)
    for c in range(n_c):
        readers = t["q_list"][t["q_ptr"][c]:t["q_ptr"][c + 1]].tolist()
        assert readers == [e for e, src in enumerate(eq) if src == c]
        writers = [e for e, w in enumerate(ew) if w == c]
        assert writers == [int(t["write_event"][c])]
        hist = t["history_list"][t["history_ptr"][c]:t["history_ptr"][c + 1]].tolist()
        assert hist == [j * 3 + i for j in range(n_q) for i in range(3) if qh[j][i] == c]
        assert (c in t["history_rows"][:-1].tolist()) == bool(hist)
    for j in range(n_q):
        assert eq[int(t["query_event"][j])] == n_c + j
    assert sorted(set(range(len(eq))) - set(plan.hidden_event.tolist())) == ep.unread_events.long().tolist()
    # the second document's conv history never reaches into the first document
    assert all(c >= 60 or c == n_c for j in range(17, n_q) for c in qh[j])
    bad = layer.cq_layer_plan(20, 3, image_groups=(4,))
    bad.event_write = bad.event_write.clone()
    bad.event_write[bad.event_write == 5] = 4  # two writers of content row 4
    with pytest.raises(ValueError, match="written by more than one event"):
        events.event_plan(bad, 4, "cpu")


def test_event_plan_fold_map_of_shared_hidden_rows():
    """A two-branch plan (Bi_I+CQ_T, ops/gated_delta_layout.py:66-83) re-writes hidden rows
    0 .. prefix-1 in its second branch: the fold map lists every distinct hidden row of
    content_order with the content rows reading it (ascending), against a direct scan; plans
    without shared rows carry no fold map; a query row may not be a content row."""
    from cqgdn import events
    import layer_harness as layer

    plan = layer.two_branch_plan(50, 12, prefix=10, suffix=15, image_groups=(6,), suffix_groups=(4,), seed=3)
    ep = events.event_plan(plan, 4, "cpu")
    t = {k: v.long() for k, v in ep.tensors.items()}
    order = plan.content_order.tolist()
    rows = sorted(set(order))
    assert ep.cstruct.n_fold_rows == len(rows) and t["fold_rows"].tolist() == rows
    for i, r in enumerate(rows):
        assert t["fold_list"][t["fold_ptr"][i]:t["fold_ptr"][i + 1]].tolist() == [c for c, x in enumerate(order)
                                                                                   if x == r]
    assert [len([c for c in order if c == r]) for r in range(10)] == [2] * 10  # the prefix, twice
    assert ep.covers_all and ep.content_bounds == (0, 50, 75)
    single = events.event_plan(layer.cq_layer_plan(30, 5, image_groups=(4,), seed=1), 4, "cpu")
    assert single.cstruct.n_fold_rows == 0
    bad = layer.cq_layer_plan(20, 3, image_groups=(4,))
    bad.query_source = bad.query_source.clone()
    bad.query_source[0] = 2  # a query reading a content row's hidden row
    with pytest.raises(ValueError, match="query rows must be distinct"):
        events.event_plan(bad, 4, "cpu")
