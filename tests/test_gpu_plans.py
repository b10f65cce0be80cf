"""GPU parity of the fused layer on plans the reference's planner builds (ops/gated_delta_layout.py:54-176),
through the restatement ``layer_harness.planner_plan`` that tests/test_planner.py pins on the CPU:

* padding positions (segment < 0): their hidden rows get no event; the layer zero-fills their outputs
  (models/backbone_qwen35.py:242-244), so those rows' outputs and, for rows that are neither content
  nor queries, their whole projection gradient are exactly zero;
* unconditional CQ queries, which read before any write of their document with an empty conv history
  (``:114-118``), queries whose target is padding (counted in document 0), and queries that no group
  reads (their rows are padding too);
* several documents with tied image groups;
* a Bi_I+CQ_T step: the masked-generation branch as a document of its own whose prefix rows write again
  without emitting, with consecutive image items forming groups (``:66-83``).

Each plan runs through ``events.layer_core`` (fwd+bwd against the float64 restatement, four seeds) and
``events.layer_prefill`` (outputs against the restatement's forward, per-document final states against
the float64 recurrence over the same event inputs).
"""

import random

import pytest
import torch

from gdn_testlib import TOL_STATE, assert_close_bf16, compare_layer, layer_parity, rel_l2
from oracle import gdn_oracle as O
from test_planner import check_plan, random_batch

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _padding_plan():
    """Three documents, 16 trailing padding positions, 70 queries (some unconditional, three aimed at
    padding positions, one of them at a group key no document has, so it is never read)."""
    rnd = random.Random(2024)
    b = random_batch(rnd, [150, 96, 64], pad=16, queries=70)
    s = len(b["sigma"])
    b["queries"][:3] = [s - 1, s - 7, s - 16]
    b["sigma"][s - 7] = 10 ** 6  # that query's group key exists in no document: nothing reads it
    b["unconditional"][3:9] = [True] * 6
    return check_plan(b)


def _generation_plan():
    """Two documents and padding, 40 queries, and a generation branch of 80 positions whose first 24
    (the prefix) re-write hidden rows 0..23 without emitting."""
    rnd = random.Random(2025)
    b = random_batch(rnd, [130, 90], pad=10, queries=40, gen=80, prefix=24)
    return check_plan(b)


PLANS = {"padding": _padding_plan, "generation": _generation_plan}


@pytest.mark.parametrize("seed", range(4))
@pytest.mark.parametrize("kind", sorted(PLANS))
def test_layer_core_on_planner_plans(gdn, kind, seed):
    plan = PLANS[kind]()
    H = 16
    pad = plan.padding_hidden
    print(f"case layer core, planner plan ({kind}): {plan.hidden_length} rows, {plan.event_q.numel()} events, "
          f"{len(plan.content_bounds) - 1} documents, {pad.numel()} padding rows, seed {seed}", flush=True)
    assert pad.numel() > 0
    gen = torch.Generator().manual_seed(300 + 1000 * seed + len(kind))
    proj = (torch.randn(plan.hidden_length, 4 * H * 128 + 2 * H, generator=gen) * 0.7).bfloat16()
    got, want, scales = layer_parity(plan, proj, H, gen)
    compare_layer(got, want, scales, H)
    out, dproj, _ = got
    out = out.detach().cpu()
    assert torch.equal(out[pad], torch.zeros_like(out[pad])), "padding rows must output zeros"
    dproj = dproj.cpu()
    live = set(plan.content_order.tolist()) | set(plan.query_source.tolist())
    dead = [r for r in pad.tolist() if r not in live]
    assert dead, "the case should hold padding rows that are neither content nor queries"
    assert torch.equal(dproj[dead], torch.zeros_like(dproj[dead])), "padding rows must get zero gradients"
    S = H * 128
    zcols = slice(3 * S, 4 * S)
    assert torch.equal(dproj[pad][:, zcols], torch.zeros_like(dproj[pad][:, zcols]))


@pytest.mark.parametrize("kind", sorted(PLANS))
def test_layer_prefill_on_planner_plans(gdn, kind):
    """layer_prefill (precise forward with final states) on the planner plans: outputs to the bf16 bar
    against the float64 restatement, padding rows exactly zero, and each document's final state
    (value-first) to the state bar against the float64 recurrence over the same event inputs (the
    restatement's q, k, v rounded to bf16, as the event pass stores them)."""
    import layer_harness as layer
    from cqgdn import events

    plan = PLANS[kind]()
    H = 16
    print(f"case layer prefill, planner plan ({kind}): {plan.hidden_length} rows", flush=True)
    gen = torch.Generator().manual_seed(400 + len(kind))
    model = layer.GatedDeltaLayer(width=64, heads=H).double()
    with torch.no_grad():
        model.conv_weight.copy_((torch.rand(model.conv_weight.shape, generator=gen) - 0.5).bfloat16().double())
        model.A_log.copy_(torch.rand(H, generator=gen).mul(3).add(0.01).log())
        model.dt_bias.copy_(torch.randn(H, generator=gen) * 0.5)
        model.norm_weight.copy_(1 + 0.1 * torch.randn(128, generator=gen))
    proj = (torch.randn(plan.hidden_length, 4 * H * 128 + 2 * H, generator=gen) * 0.7).bfloat16()
    params = [model.conv_weight.bfloat16(), model.A_log.float(), model.dt_bias.float(), model.norm_weight.float()]
    out, cache = events.layer_prefill(proj.to(DEV), *(p.detach().to(DEV) for p in params), plan, heads=H)
    torch.cuda.synchronize()
    states = {}

    def recurrence(q, k, v, g, b, p):
        # the states against the recurrence over the event inputs the kernels consume: q, k, v rounded
        # to bf16 by the event pass (g and beta are fp32 there)
        r = lambda t: t.bfloat16().double()
        states["final"] = O.chunk_delta(r(q), r(k), r(v), g, b, p.event_bounds, normalize=True,
                                        output_final_state=True)[1]
        return O.chunk_delta(q, k, v, g, b, p.event_bounds, normalize=True)

    with torch.no_grad():
        ref = model.core(proj.double(), plan, recurrence=recurrence,
                         conv=lambda u, w, bounds: O.causal_conv1d(u, w, bounds), norm=O.gated_rms_norm, fused=False)
    out = out.cpu()
    assert_close_bf16("out", out, ref)
    pad = plan.padding_hidden
    assert torch.equal(out[pad], torch.zeros_like(out[pad]))
    want = states["final"].transpose(-1, -2)
    got = cache["state"].cpu()
    assert got.shape == want.shape, (got.shape, want.shape)
    for d in range(got.shape[0]):
        r = rel_l2(got[d], want[d])
        print(f"  state of document {d}: rel_l2={r:.3e}", flush=True)
        assert r <= TOL_STATE
