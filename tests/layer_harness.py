"""Test and benchmark harness: a whole GatedDelta layer and DeltaPlans to drive it.

Nothing in the drop-in path imports this module; the tests and ``bench.py`` do.

* ``GatedDeltaLayer`` is the whole layer the reference's layer benchmark times at
  width 2048 (scripts/benchmark_gdn.py:34-56): fused input projection, causal conv
  over the content, the CQ query conv from the content history, the event gathers,
  the gates, the recurrence, the output gather with the padding fill, gated RMSNorm
  and out_proj (models/backbone_qwen35.py:156-246, the training path without a state
  cache).  By default everything between the two projections runs in the fused
  kernels of ``events.layer_core``; ``core(..., fused=False)`` is the reference's
  layer code restated around hooks for the conv, the recurrence and the norm, which
  the parity tests fill with the float64 oracle.
* ``planner_plan`` builds the DeltaPlan the reference's planner
  (ops/gated_delta_layout.py:54-176) builds for a described microbatch: documents,
  padding positions, sigma groups, CQ queries (conditional or not) and the
  masked-generation branch.  ``cq_layer_plan``, ``two_branch_plan`` and
  ``concat_plans`` build synthetic plans of the same structure at benchmark sizes.
"""

from __future__ import annotations

import random
from dataclasses import dataclass, fields

import torch
import torch.nn.functional as F

from cqgdn import events
from cqgdn import gated_delta_net as gdn


@dataclass
class LayerPlan:
    """The reference's DeltaPlan (ops/gated_delta_layout.py:12-27), field for field."""

    content_order: torch.Tensor  # hidden row of each content write, in write order
    event_q: torch.Tensor  # per event: row of cat(content q, query q)
    event_write: torch.Tensor  # per event: content row it writes, or n_content (zero row: read-only)
    query_source: torch.Tensor  # hidden row of each query
    query_history: torch.Tensor  # [n_queries, kernel - 1] content rows of the query conv (n_content = none)
    content_cu: torch.Tensor
    content_bounds: tuple
    event_cu: torch.Tensor
    event_bounds: tuple
    hidden_length: int
    hidden_event: torch.Tensor  # per hidden row: the event whose output it takes (0 for padding rows)
    output_event: torch.Tensor = None  # emitting events, in event order
    output_hidden: torch.Tensor = None  # the hidden row each of them feeds
    padding_hidden: torch.Tensor = None  # hidden rows no event feeds; their outputs are zero

    def __post_init__(self):
        if self.output_event is None:  # every hidden row emits (the synthetic plans)
            order = torch.argsort(self.hidden_event)
            self.output_event = self.hidden_event[order]
            self.output_hidden = order
            self.padding_hidden = torch.zeros(0, dtype=torch.long)

    def to(self, device):
        return LayerPlan(**{f.name: (getattr(self, f.name).to(device) if isinstance(getattr(self, f.name), torch.Tensor)
                                     else getattr(self, f.name)) for f in fields(self)})


def planner_plan(sigma, segments, queries=(), unconditional=None, generation=(), prefix=0, generation_image=(),
                 kernel=4) -> LayerPlan:
    """The plan ops/gated_delta_layout.py:54-176 builds for one microbatch (B = 1), described by:

    * ``sigma[i]``, ``segments[i]``: the write order key and the document of content position i
      (segment < 0: a padding position; it is neither written nor read, and its hidden row is padding);
    * ``queries``: the target position of each CQ query (hidden row ``keys + j``); ``unconditional[j]``
      marks a query that reads before any write of its document, with an empty conv history
      (``:86-95``, ``:114-118``).  A query whose target sits in padding is counted in document 0
      (``:92-93``); one whose document or sigma group has no content is never read (its row is padding);
    * ``generation``, ``prefix``, ``generation_image``: the masked-generation branch of a Bi_I+CQ_T step
      (``:66-83``).  Its items are the generation positions in their own group order (consecutive
      image items form one group); the first ``prefix`` items write hidden rows 0 .. prefix-1 again
      without emitting, the rest are new rows ``len(sigma) ..``.

    Events: per branch, per document in order of first appearance, per group in ascending key:
    the group's queries (branch 0 only, each a read-only event), then each member's write, then,
    for a multi-member group, one read-only re-read per member, which carries the member's output.
    """
    s = len(sigma)
    suffix = len(generation) - prefix if len(generation) else 0
    keys = s + suffix
    unconditional = list(unconditional) if unconditional is not None else [False] * len(queries)
    main = [(i, segments[i], sigma[i], True) for i in range(s) if segments[i] >= 0]
    branches = [main]
    if len(generation):
        keys_of, key, prev_image = [], -1, False
        for image in generation_image:
            key += 0 if (image and prev_image) else 1
            keys_of.append(key)
            prev_image = image
        branches.append([(i if i < prefix else s + i - prefix, segments[p], keys_of[i], i >= prefix)
                         for i, p in enumerate(generation) if segments[p] >= 0])
    if not branches[0]:
        branches[0] = [(0, 0, 0, True)]  # an all-padding microbatch still has one written row
    # queries by document, then by the group key they read before (None: before every group)
    attached = {}
    for j, p in enumerate(queries):
        doc = max(segments[p], 0)
        attached.setdefault(doc, {}).setdefault(None if unconditional[j] else sigma[p], []).append(keys + j)
    order, reads, writes, emit_event, emit_hidden, q_rows, q_hist = [], [], [], [], [], [], []
    c_bounds, e_bounds = [0], [0]

    def add_event(read, write, out_row=None):
        reads.append(read)
        writes.append(write)
        if out_row is not None:
            emit_event.append(len(reads) - 1)
            emit_hidden.append(out_row)

    for b, items in enumerate(branches):
        docs = {}
        for item in items:
            docs.setdefault(item[1], []).append(item)
        for doc, members in docs.items():
            groups = {}
            for item in sorted(members, key=lambda it: (it[2], it[0])):
                groups.setdefault(item[2], []).append(item)
            pending = dict(attached.get(doc, {})) if b == 0 else {}
            if None in pending:
                first = next(iter(groups))
                pending[first] = pending.pop(None) + pending.get(first, [])
            written = []  # this document's content rows so far (the query conv's history)
            for key, group in groups.items():
                for row in pending.get(key, []):
                    hist = written[-(kernel - 1):] if kernel > 1 else []
                    q_hist.append([None] * (kernel - 1 - len(hist)) + hist)
                    q_rows.append(row)
                    add_event(("q", len(q_rows) - 1), None, row)
                idx = []
                for hidden_row, _, _, emits in group:
                    ci = len(order)
                    order.append(hidden_row)
                    idx.append((ci, hidden_row, emits))
                    written.append(ci)
                    add_event(("c", ci), ci, hidden_row if (len(group) == 1 and emits) else None)
                if len(group) > 1:
                    for ci, hidden_row, emits in idx:
                        add_event(("c", ci), None, hidden_row if emits else None)
            c_bounds.append(len(order))
            e_bounds.append(len(reads))
    nc, n_h = len(order), keys + len(queries)
    long = lambda xs: torch.tensor(xs, dtype=torch.long)
    hidden_event = torch.zeros(n_h, dtype=torch.long)
    hidden_event[long(emit_hidden)] = long(emit_event)
    padding = torch.ones(n_h, dtype=torch.bool)
    padding[long(emit_hidden)] = False
    return LayerPlan(
        content_order=long(order),
        event_q=long([i if kind == "c" else nc + i for kind, i in reads]),
        event_write=long([nc if w is None else w for w in writes]),
        query_source=long(q_rows),
        query_history=long([[nc if c is None else c for c in h] for h in q_hist]).reshape(len(q_rows), kernel - 1),
        content_cu=torch.tensor(c_bounds, dtype=torch.int32),
        content_bounds=tuple(c_bounds),
        event_cu=long(e_bounds),
        event_bounds=tuple(e_bounds),
        hidden_length=n_h,
        hidden_event=hidden_event,
        output_event=long(emit_event),
        output_hidden=long(emit_hidden),
        padding_hidden=padding.nonzero().flatten(),
    )


def cq_layer_plan(content: int, queries: int, image_groups=(249, 249), kernel: int = 4, seed: int = 0) -> LayerPlan:
    """One document of ``content`` tokens (image groups at seeded positions, text tokens
    as single-token groups) and ``queries`` read-only CQ queries attached to seeded
    groups.  Events: content + queries + sum(image_groups)."""
    rnd = random.Random(seed)
    # image groups: disjoint runs of consecutive content positions
    starts, free = [], content
    for size in image_groups:
        free -= size
    cuts = sorted(rnd.sample(range(free + 1), len(image_groups)))
    offset = 0
    for cut, size in zip(cuts, image_groups):
        starts.append(cut + offset)
        offset += size
    groups, pos = [], 0
    image_at = dict(zip(starts, image_groups))
    while pos < content:
        size = image_at.get(pos, 1)
        groups.append(list(range(pos, pos + size)))
        pos += size
    attach = {}
    for j in range(queries):
        attach.setdefault(rnd.randrange(len(groups)), []).append(j)

    nc = content
    event_q, event_write, out_event = [], [], {}
    query_history, history = [None] * queries, []
    for gi, members in enumerate(groups):
        for j in attach.get(gi, []):
            prev = history[-(kernel - 1):] if kernel > 1 else []
            query_history[j] = [nc] * (kernel - 1 - len(prev)) + prev
            out_event[content + j] = len(event_q)
            event_q.append(nc + j)
            event_write.append(nc)
        for ci in members:
            if len(members) == 1:
                out_event[ci] = len(event_q)
            event_q.append(ci)
            event_write.append(ci)
            history.append(ci)
        if len(members) > 1:
            for ci in members:
                out_event[ci] = len(event_q)
                event_q.append(ci)
                event_write.append(nc)
    hidden = content + queries
    long = lambda xs: torch.tensor(xs, dtype=torch.long)
    events = len(event_q)
    return LayerPlan(
        content_order=torch.arange(content),
        event_q=long(event_q),
        event_write=long(event_write),
        query_source=torch.arange(content, hidden),
        query_history=long(query_history).reshape(queries, kernel - 1),
        content_cu=torch.tensor([0, content], dtype=torch.int32),
        content_bounds=(0, content),
        event_cu=torch.tensor([0, events], dtype=torch.long),
        event_bounds=(0, events),
        hidden_length=hidden,
        hidden_event=long([out_event[r] for r in range(hidden)]),
    )


def two_branch_plan(content: int, queries: int, prefix: int, suffix: int, image_groups=(), suffix_groups=(8,),
                    kernel: int = 4, seed: int = 0) -> LayerPlan:
    """A plan with the two branches of a Bi_I+CQ_T step (ops/gated_delta_layout.py:55-83, 108-150).

    Branch 0 is ``cq_layer_plan(content, queries, image_groups)``: hidden rows 0 .. content-1
    plus the queries.  Branch 1, the masked-generation branch, is a document of its own whose
    first ``prefix`` items re-write hidden rows 0 .. prefix-1 (without emitting outputs, as the
    reference's ``i >= plan.prefix`` flag) and whose ``suffix`` items are new hidden rows
    content .. content+suffix-1, with multi-token groups of ``suffix_groups`` sizes at seeded
    places.  Query hidden rows follow all keys (keys + j).  So content_order repeats hidden rows
    0 .. prefix-1, and the layer's backward must sum their gradients."""
    base = cq_layer_plan(content, queries, image_groups, kernel, seed)
    rnd = random.Random(seed + 1)
    keys = content + suffix
    n1 = prefix + suffix
    hidden1 = list(range(prefix)) + list(range(content, keys))
    emit1 = [False] * prefix + [True] * suffix
    # groups of branch 1: single tokens, and the multi-token groups placed in the suffix
    sizes, pos, groups = list(suffix_groups), 0, []
    starts = sorted(rnd.sample(range(prefix, n1 - sum(sizes) + 1), len(sizes))) if sizes else []
    shift, at = 0, {}
    for st, size in zip(starts, sizes):
        at[st + shift] = size
        shift += size
    while pos < n1:
        size = at.get(pos, 1)
        groups.append(list(range(pos, pos + size)))
        pos += size
    nc = content + n1
    ev0 = base.event_q.numel()
    q0 = base.event_q.clone()
    eq0 = torch.where(q0 < content, q0, q0 - content + nc)  # query rows move past branch 1's content rows
    ew0 = torch.where(base.event_write < content, base.event_write, torch.full_like(base.event_write, nc))
    event_q, event_write, out = [], [], {}
    for members in groups:
        for i in members:
            ci = content + i
            if len(members) == 1 and emit1[i]:
                out[hidden1[i]] = ev0 + len(event_q)
            event_q.append(ci)
            event_write.append(ci)
        if len(members) > 1:
            for i in members:
                if emit1[i]:
                    out[hidden1[i]] = ev0 + len(event_q)
                event_q.append(content + i)
                event_write.append(nc)
    hidden_event = torch.empty(keys + queries, dtype=torch.long)
    hidden_event[:content] = base.hidden_event[:content]
    for r, e in out.items():
        hidden_event[r] = e
    hidden_event[keys:] = base.hidden_event[content:]
    qh = base.query_history
    long = lambda xs: torch.tensor(xs, dtype=torch.long)
    n_events = ev0 + len(event_q)
    return LayerPlan(
        content_order=torch.cat((base.content_order, long(hidden1))),
        event_q=torch.cat((eq0, long(event_q))),
        event_write=torch.cat((ew0, long(event_write))),
        query_source=torch.arange(keys, keys + queries),
        query_history=torch.where(qh < content, qh, torch.full_like(qh, nc)),
        content_cu=torch.tensor([0, content, nc], dtype=torch.int32),
        content_bounds=(0, content, nc),
        event_cu=torch.tensor([0, ev0, n_events], dtype=torch.long),
        event_bounds=(0, ev0, n_events),
        hidden_length=keys + queries,
        hidden_event=hidden_event,
    )


def concat_plans(*plans: LayerPlan) -> LayerPlan:
    """Pack single-document plans into one plan of several documents (the layout
    ops/gated_delta_layout.py:105-150 produces for a packed batch): hidden rows, content
    rows, queries and events of each plan follow those of the plans before it."""
    n_c = sum(len(p.content_order) for p in plans)
    n_q = sum(len(p.query_source) for p in plans)
    fields = {k: [] for k in ("content_order", "event_q", "event_write", "query_source", "query_history",
                              "hidden_event")}
    cb, eb = [0], [0]
    h0 = c0 = q0 = e0 = 0
    for p in plans:
        pc, pq, pe = len(p.content_order), len(p.query_source), len(p.event_q)
        content = lambda t: torch.where(t < pc, t + c0, torch.full_like(t, n_c))
        fields["content_order"].append(p.content_order + h0)
        fields["event_q"].append(torch.where(p.event_q < pc, p.event_q + c0, p.event_q - pc + n_c + q0))
        fields["event_write"].append(content(p.event_write))
        fields["query_source"].append(p.query_source + h0)
        fields["query_history"].append(content(p.query_history))
        fields["hidden_event"].append(p.hidden_event + e0)
        h0, c0, q0, e0 = h0 + p.hidden_length, c0 + pc, q0 + pq, e0 + pe
        cb.append(c0)
        eb.append(e0)
    cat = {k: torch.cat(v) for k, v in fields.items()}
    return LayerPlan(content_cu=torch.tensor(cb, dtype=torch.int32), content_bounds=tuple(cb),
                     event_cu=torch.tensor(eb, dtype=torch.long), event_bounds=tuple(eb), hidden_length=h0, **cat)


class GatedDeltaLayer(torch.nn.Module):
    """GatedDelta with fused projections (models/backbone_qwen35.py:121-154), one TP rank."""

    def __init__(self, width=2048, heads=16, head_dim=128, conv_kernel=4, eps=1e-6, key_heads=None):
        super().__init__()
        # heads: value heads (linear_value_heads); key_heads: q/k heads (linear_heads), default heads
        self.key_heads = heads if key_heads is None else key_heads
        self.heads, self.head_dim, self.kernel = heads, head_dim, conv_kernel
        key, value = self.key_heads * head_dim, heads * head_dim
        self.in_proj_all = torch.nn.Linear(width, 2 * key + 2 * value + 2 * heads, bias=False)
        self.conv_weight = torch.nn.Parameter(torch.empty(2 * key + value, conv_kernel).uniform_(-0.5, 0.5))
        self.A_log = torch.nn.Parameter(torch.rand(heads).mul(15.99).add(0.01).log())
        self.dt_bias = torch.nn.Parameter(torch.ones(heads))
        self.norm_weight = torch.nn.Parameter(torch.ones(head_dim))
        self.out_proj = torch.nn.Linear(value, width, bias=False)
        self.eps = eps
        for lin in (self.in_proj_all, self.out_proj):
            torch.nn.init.normal_(lin.weight, std=0.02)

    def forward(self, x, plan: LayerPlan, recurrence=None, conv=None, norm=None, fused=True):
        """x [rows, 1, width] -> [rows, 1, width].  See ``core`` for the hooks and ``fused``."""
        proj = self.in_proj_all(x[:, 0])
        return self.out_proj(self.core(proj, plan, recurrence, conv, norm, fused))[:, None]

    def core(self, proj, plan: LayerPlan, recurrence=None, conv=None, norm=None, fused=True):
        """Everything between the projections: proj [rows, 2SK + 2SV + 2H] -> gated-norm rows [rows, SV].

        With ``fused`` and no hooks this is ``events.layer_core`` (the fused HIP kernels).
        Otherwise it is the reference's torch code with the hip delta, conv and gated norm, which
        ``recurrence(q, k, v, g, beta, plan)``, ``conv(x, weight, bounds)`` and
        ``norm(y, z, weight, eps)`` replace when given (tests pass float64 CPU restatements)."""
        h, hk, d = self.heads, self.key_heads, self.head_dim
        size, vsize = hk * d, h * d
        if fused and recurrence is None and conv is None and norm is None:
            return events.layer_core(proj, self.conv_weight, self.A_log, self.dt_bias, self.norm_weight, plan,
                                     heads=h, key_heads=hk, eps=self.eps)
        raw, z, a, beta = proj.split((2 * size + vsize, vsize, h, h), -1)
        updates = raw.index_select(0, plan.content_order)
        if conv is None:
            convolved = gdn.conv(updates[None], self.conv_weight, activation="silu", cu_seqlens=plan.content_cu,
                                 cu_seqlens_cpu=plan.content_bounds)[0][0]
        else:
            convolved = conv(updates[None], self.conv_weight, plan.content_bounds)[0]
        q, k, v = convolved.split((size, size, vsize), -1)
        q, k, v = q.reshape(-1, hk, d), k.reshape(-1, hk, d), v.reshape(-1, h, d)
        # the CQ query conv reads the content history only
        raw_q = raw[:, :size].index_select(0, plan.query_source)
        weight = self.conv_weight[:size]
        query = raw_q * weight[:, -1]
        history = torch.cat((updates[:, :size], updates.new_zeros(1, size)), dim=0)
        for j in range(self.kernel - 1):
            query = query + history.index_select(0, plan.query_history[:, j]) * weight[:, j]
        query = F.silu(query).reshape(-1, hk, d)
        if h != hk:
            q, k, query = (t.repeat_interleave(h // hk, dim=1) for t in (q, k, query))
        q = torch.cat((q, query), dim=0).index_select(0, plan.event_q)[None]
        zeros = k.new_zeros(1, h, d)
        k = torch.cat((k, zeros), dim=0).index_select(0, plan.event_write)[None]
        v = torch.cat((v, zeros), dim=0).index_select(0, plan.event_write)[None]
        control = torch.float64 if proj.dtype == torch.float64 else torch.float32
        a = a.index_select(0, plan.content_order).to(control)
        g = -self.A_log.to(control).exp() * F.softplus(a + self.dt_bias.to(control))
        beta = beta.index_select(0, plan.content_order).sigmoid().to(control)
        control_zero = g.new_zeros(1, h)
        g = torch.cat((g, control_zero)).index_select(0, plan.event_write)[None]
        beta = torch.cat((beta, control_zero)).index_select(0, plan.event_write)[None]
        if recurrence is None:
            y = gdn.delta(q, k, v, g, beta, use_qk_l2norm_in_kernel=True, cu_seqlens=plan.event_cu,
                          cu_seqlens_cpu=plan.event_bounds)[0]
        else:
            y = recurrence(q, k, v, g, beta, plan)
        selected = y[0].index_select(0, plan.hidden_event).to(proj.dtype)
        if plan.padding_hidden is not None and plan.padding_hidden.numel():
            selected.index_fill_(0, plan.padding_hidden, 0)
        if norm is None:
            out = gdn.gated_norm(selected, z.reshape(-1, h, d), self.norm_weight, self.eps)
        else:
            out = norm(selected, z.reshape(-1, h, d), self.norm_weight, self.eps)
        return out.flatten(-2)
