"""The harness's restatement of the reference planner (ops/gated_delta_layout.py:54-176), pinned by the
CQ semantics its module docstring states rather than by its own steps:

* within a document, content writes follow (sigma, position) order;
* a tied image group is fully written before any of its members' outputs;
* a CQ query reads before its target's sigma group, with the conv history of the content written
  before it; an unconditional query reads before any write, with an empty history (``:114-118``);
* read-only events leave the state alone, and padding rows get no output (``:155-158``);
* the masked-generation branch is a document of its own whose prefix rows write without emitting.

Each case is checked by recomputing, for every hidden row, which content rows its output sees and in
what order, directly from the batch description, and comparing with the writes the plan's events
perform before that row's output event.  Then ``events.event_plan`` must accept the plan (padding
rows read nothing), and the float64 layer restatement must give padding rows a zero output and,
for rows that are neither content nor queries, a zero projection gradient.
"""

import random

import pytest
import torch

import layer_harness as L
from cqgdn import events


def random_batch(rnd, docs, pad, queries, gen=0, prefix=0):
    """A microbatch description: ``docs`` document lengths, ``pad`` trailing padding positions,
    sigma keys with tied image groups at random places, ``queries`` CQ targets (some in padding,
    some unconditional), and a generation branch of ``gen`` positions with ``prefix``."""
    sigma, segments = [], []
    for d, n in enumerate(docs):
        # groups: mostly single tokens, a few image groups of 2-5 tokens, at shuffled places
        sizes = []
        while sum(sizes) < n:
            sizes.append(min(n - sum(sizes), rnd.choice([1, 1, 1, 2, 3, 5])))
        keys = list(range(len(sizes)))
        rnd.shuffle(keys)
        flat = [k for k, size in zip(keys, sizes) for _ in range(size)]
        rnd.shuffle(flat)
        sigma += flat
        segments += [d] * n
    sigma += [0] * pad
    segments += [-1] * pad
    s = len(sigma)
    q = [rnd.randrange(s) for _ in range(queries)]
    unconditional = [rnd.random() < 0.25 for _ in range(queries)]
    generation = sorted(rnd.sample(range(s), gen)) if gen else []
    gimage = [rnd.random() < 0.4 for _ in range(gen)]
    return dict(sigma=sigma, segments=segments, queries=q, unconditional=unconditional, generation=generation,
                prefix=prefix, generation_image=gimage)


def expected_views(b, kernel=4):
    """For every emitted hidden row: (branch, document, the hidden rows it sees in write order, and for a
    query its history rows), computed from the description alone."""
    sigma, seg, s = b["sigma"], b["segments"], len(b["sigma"])
    gen, prefix = b["generation"], b["prefix"]
    suffix = len(gen) - prefix if gen else 0
    keys = s + suffix
    items = {}  # (branch, doc) -> list of (key, hidden row, emits)
    for i in range(s):
        if seg[i] >= 0:
            items.setdefault((0, seg[i]), []).append((sigma[i], i, True))
    if not any(k[0] == 0 for k in items):
        items[(0, 0)] = [(0, 0, True)]
    group, prev = -1, False
    for i, p in enumerate(gen):
        image = b["generation_image"][i]
        group += 0 if (image and prev) else 1
        prev = image
        if seg[p] >= 0:
            items.setdefault((1, seg[p]), []).append((group, i if i < prefix else s + i - prefix, i >= prefix))
    views = {}
    for (br, doc), its in items.items():
        its = sorted(its)
        for key, row, emits in its:
            if emits:
                views[row] = (br, doc, [r for k, r, _ in its if k <= key], None)
    for j, p in enumerate(b["queries"]):
        doc = max(seg[p], 0)
        its = sorted(items.get((0, doc), []))
        if not its:
            continue
        if b["unconditional"][j]:
            seen = []
        else:
            if sigma[p] not in {k for k, _, _ in its}:
                continue  # no group of that key in the document: never read
            seen = [r for k, r, _ in its if k < sigma[p]]
        views[keys + j] = (0, doc, seen, seen[-(kernel - 1):])
    return views, keys + len(b["queries"])


def plan_views(plan):
    """The same views, read off the plan's events."""
    order, eq, ew = plan.content_order.tolist(), plan.event_q.tolist(), plan.event_write.tolist()
    nc, bounds = len(order), plan.event_bounds
    qs, qh = plan.query_source.tolist(), plan.query_history.tolist()
    views = {}
    for e, row in zip(plan.output_event.tolist(), plan.output_hidden.tolist()):
        d = max(i for i in range(len(bounds) - 1) if bounds[i] <= e)
        seen = [order[w] for w in ew[bounds[d]:e + 1] if w < nc]
        if eq[e] < nc:
            assert order[eq[e]] == row, "a content output reads another row's q"
            views[row] = (d, seen, None)
        else:
            j = eq[e] - nc
            assert qs[j] == row and ew[e] == nc
            views[row] = (d, seen, [order[c] for c in qh[j] if c < nc])
    return views


def check_plan(b, kernel=4):
    plan = L.planner_plan(**b, kernel=kernel)
    want, n_h = expected_views(b, kernel)
    got = plan_views(plan)
    assert plan.hidden_length == n_h
    assert sorted(got) == sorted(want), "emitted rows differ"
    # documents in event order: branch 0's documents, then branch 1's
    doc_index = {}
    for row, (br, doc, seen, hist) in sorted(want.items(), key=lambda kv: plan.hidden_event[kv[0]].item()):
        doc_index.setdefault((br, doc), len(doc_index))
    for row, (br, doc, seen, hist) in want.items():
        d, pseen, phist = got[row]
        assert pseen == seen, f"row {row}: sees {pseen}, expected {seen}"
        assert phist == hist, f"row {row}: history {phist}, expected {hist}"
    # queries that read at the same point keep the planner's order: unconditional ones first, then
    # by query index (invisible to every value, but part of the plan's layout)
    nc, qs = plan.content_order.numel(), plan.query_source.tolist()
    keys = len(b["sigma"]) + (len(b["generation"]) - b["prefix"] if b["generation"] else 0)
    eq, starts, run = plan.event_q.tolist(), set(plan.event_bounds), []
    for e in range(len(eq) + 1):
        if e == len(eq) or e in starts or eq[e] < nc:
            assert run == sorted(run), f"queries out of order: {run}"
            run = []
        if e < len(eq) and eq[e] >= nc:
            j = qs[eq[e] - nc] - keys
            run.append((not b["unconditional"][j], j))
    pad = sorted(set(range(n_h)) - set(want))
    assert plan.padding_hidden.tolist() == pad
    assert all(plan.hidden_event[r] == 0 for r in pad)
    # read-only events write nothing; every content row is written exactly once
    nc = plan.content_order.numel()
    writes = [w for w in plan.event_write.tolist() if w < nc]
    assert sorted(writes) == list(range(nc))
    return plan


@pytest.mark.parametrize("seed", range(12))
def test_planner_semantics_random_batches(seed):
    rnd = random.Random(seed)
    docs = [rnd.randint(1, 30) for _ in range(rnd.randint(1, 4))]
    gen = rnd.choice([0, 0, 6, 11])
    b = random_batch(rnd, docs, pad=rnd.choice([0, 3, 9]), queries=rnd.randint(0, 14), gen=gen,
                     prefix=rnd.randint(0, gen // 2) if gen else 0)
    plan = check_plan(b)
    ep = events.event_plan(plan, 4, "cpu")
    hidden = ep.hidden_index.tolist()
    assert all(hidden[r] == -1 for r in plan.padding_hidden.tolist())
    assert sorted(h for h in hidden if h >= 0) == sorted(plan.output_event.tolist())


def test_planner_pure_text_is_causal():
    """One document, sigma = positions, no queries: the plan is the plain causal stream
    (the setting of the reference's tests/test_qwen35_cq.py:53-58)."""
    plan = check_plan(dict(sigma=list(range(17)), segments=[0] * 17, queries=[], unconditional=[], generation=[],
                           prefix=0, generation_image=[]))
    ar = torch.arange(17)
    for t in (plan.content_order, plan.event_q, plan.event_write, plan.hidden_event, plan.output_event):
        assert torch.equal(t, ar)
    assert plan.padding_hidden.numel() == 0 and plan.event_bounds == (0, 17)


def test_planner_all_padding_keeps_one_row():
    """A microbatch with no content still plans one written row (the zero-loss EOF graph, :84-85)."""
    plan = check_plan(dict(sigma=[0, 0, 0], segments=[-1, -1, -1], queries=[1], unconditional=[False], generation=[],
                           prefix=0, generation_image=[]))
    assert plan.content_order.tolist() == [0] and plan.padding_hidden.tolist() == [1, 2]


def test_restatement_zeroes_padding_rows():
    """The float64 layer restatement on a planner plan with padding: padding rows' outputs are exactly
    zero (models/backbone_qwen35.py:242-244), and so is the whole projection gradient of padding rows
    that are neither content nor query rows."""
    from oracle import gdn_oracle as O

    rnd = random.Random(5)
    b = random_batch(rnd, [14, 9], pad=5, queries=6)
    b["queries"][0] = len(b["sigma"]) - 1  # one query aimed at a padding position
    plan = L.planner_plan(**b)
    assert plan.padding_hidden.numel() >= 5
    H = 4
    model = L.GatedDeltaLayer(width=32, heads=H).double()
    gen = torch.Generator().manual_seed(3)
    proj = (torch.randn(plan.hidden_length, 4 * H * 128 + 2 * H, generator=gen) * 0.7).double().requires_grad_()
    rec = lambda q, k, v, g, bb, p: O.recurrent_delta(q, k, v, g, bb, p.event_bounds, normalize=True)
    cv = lambda u, w, bounds: O.causal_conv1d(u, w, bounds)
    out = model.core(proj, plan, recurrence=rec, conv=cv, norm=O.gated_rms_norm, fused=False)
    out.backward(torch.randn(out.shape, generator=gen, dtype=torch.float64))
    pad = plan.padding_hidden
    assert torch.equal(out[pad], torch.zeros_like(out[pad]))
    live = set(plan.content_order.tolist()) | set(plan.query_source.tolist())
    dead = [r for r in pad.tolist() if r not in live]
    assert dead and torch.equal(proj.grad[dead], torch.zeros_like(proj.grad[dead]))
