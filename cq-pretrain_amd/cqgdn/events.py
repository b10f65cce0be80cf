"""One GatedDelta layer between its two projections, on the GPU (models/backbone_qwen35.py:158-246).

``layer_core`` does what the reference's ``GatedDelta.forward`` does between
``in_proj_all`` and ``out_proj``: the content gather and packed causal conv, the CQ
query conv from the content history, the q/k/v/g/beta event gathers and the gate
math, the recurrence, the output gather and the gated RMSNorm.  It takes the fused
projection as one [rows, 2SK + 2SV + 2H] tensor (H value heads, HK key heads,
SK = HK * 128, SV = H * 128; columns q|k|v, z, a, b as ``in_proj_all(...).split``
lays them out) and returns the normalized [rows, SV] rows for ``out_proj``.  With
fewer key heads than value heads, value head j reads key head j // (H // HK), as
the reference's repeat_interleave does (models/backbone_qwen35.py:182-183).  Forward: cqgdn_event_inputs_fwd (the conv pass and the event
pass), the recurrence, cqgdn_gated_norm_fwd.  Backward: the norm, the recurrence and
cqgdn_event_inputs_bwd write one projection-gradient tensor, each element once:
every gather of the reference is consumed inside a kernel's loads, and every
scatter-add of its autograd (index_select backward) is replaced by a walk over an
inverse map, deterministic and without atomics.

``event_plan`` derives the device index arrays and the inverse maps of a plan once
and keeps them on the plan (one plan serves every layer of a step).
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import torch

from . import _lib
from . import gated_delta_net as gdn


@dataclass
class EventPlan:
    """Device int32 index arrays of one plan for the fused layer kernels."""

    device: str
    kernel: int
    n_hidden: int
    n_content: int
    n_queries: int
    n_events: int
    content_bounds: tuple
    event_bounds: tuple
    hidden_index: torch.Tensor  # [n_hidden] event each hidden row reads, -1 for padding rows
    unread_events: torch.Tensor  # events no hidden row reads (their output gradient is zero)
    covers_all: bool  # every hidden row is a content or a query row
    tensors: dict = field(default_factory=dict)
    cstruct: _lib.EventPlan = None


def _csr(keys, values, n):
    """Entries grouped by key (0 .. n-1), values in their input order within a key."""
    idx = torch.sort(keys, stable=True).indices
    ptr = torch.zeros(n + 1, dtype=torch.long)
    ptr[1:] = torch.bincount(keys, minlength=n).cumsum(0)
    return ptr, values[idx]


def _check(cond, msg):
    if not cond:
        raise ValueError(f"invalid event plan: {msg}")


def event_plan(plan, kernel: int, device) -> EventPlan:
    """The plan's index arrays and inverse maps on ``device``, built once per plan.

    ``plan`` carries the DeltaPlan fields the layer reads (ops/gated_delta_layout.py:13-27):
    content_order, event_q, event_write, query_source, query_history, content_bounds,
    event_bounds, hidden_length, hidden_event and, optionally, padding_hidden.
    """
    device = str(device)
    cached = getattr(plan, "_cqgdn_event_plan", None)
    if cached is not None and cached.device == device and cached.kernel == kernel:
        return cached
    cpu = lambda t: t.detach().to("cpu", torch.long)
    order, eq, ew, qs = cpu(plan.content_order), cpu(plan.event_q), cpu(plan.event_write), cpu(plan.query_source)
    n_c, n_q, n_e, n_h = order.numel(), qs.numel(), eq.numel(), int(plan.hidden_length)
    qh = cpu(plan.query_history).reshape(n_q, kernel - 1)
    _check(2 <= kernel <= 4, "conv kernel must be 2..4")
    _check(ew.numel() == n_e, "event_q and event_write differ in length")
    rows = torch.cat((order, qs))
    _check(rows.numel() == 0 or (rows.min() >= 0 and rows.max() < n_h), "content/query rows outside the hidden rows")
    # Content rows may share a hidden row: Bi_I+CQ_T plans write the generation prefix's
    # rows again in their second branch (ops/gated_delta_layout.py:66-83).  Queries read
    # rows of their own.
    content_rows = torch.unique(order)
    _check(torch.unique(qs).numel() == n_q and torch.unique(torch.cat((content_rows, qs))).numel() ==
           content_rows.numel() + n_q, "query rows must be distinct from each other and from content rows")
    _check(n_e == 0 or (eq.min() >= 0 and eq.max() < n_c + n_q), "event_q out of range")
    _check(n_e == 0 or (ew.min() >= 0 and ew.max() <= n_c), "event_write out of range")
    _check(qh.numel() == 0 or (qh.min() >= 0 and qh.max() <= n_c), "query_history out of range")
    _check(tuple(plan.content_bounds)[-1] == n_c and tuple(plan.event_bounds)[-1] == n_e, "bounds do not cover rows")
    events = torch.arange(n_e)
    qmask, wmask = eq < n_c, ew < n_c
    _check(torch.equal(torch.bincount(eq[~qmask] - n_c, minlength=n_q), torch.ones(n_q, dtype=torch.long)),
           "every query must be read by exactly one event")
    _check(n_c == 0 or int(torch.bincount(ew[wmask], minlength=n_c).max()) <= 1,
           "a content row is written by more than one event")
    q_ptr, q_list = _csr(eq[qmask], events[qmask], n_c)
    write_event = torch.full((n_c,), -1, dtype=torch.long)
    write_event[ew[wmask]] = events[wmask]
    query_event = torch.empty(n_q, dtype=torch.long)
    query_event[eq[~qmask] - n_c] = events[~qmask]
    flat = qh.flatten()
    hmask = flat < n_c
    h_ptr, h_list = _csr(flat[hmask], torch.arange(flat.numel())[hmask], n_c)
    h_rows = torch.nonzero(h_ptr[1:] > h_ptr[:-1]).flatten()
    hidden = cpu(plan.hidden_event).clone()
    padding = getattr(plan, "padding_hidden", None)
    if padding is not None and padding.numel():
        hidden[cpu(padding)] = -1
    _check(hidden.numel() == n_h and (n_h == 0 or (hidden.min() >= -1 and hidden.max() < n_e)),
           "hidden_event out of range")
    real = hidden[hidden >= 0]
    _check(torch.unique(real).numel() == real.numel(), "two hidden rows read the same event")
    read = torch.zeros(n_e, dtype=torch.bool)
    read[real] = True
    shared = content_rows.numel() < n_c
    if shared:  # hidden row -> the content rows reading it, ascending (the backward sums them)
        slot = torch.searchsorted(content_rows, order)
        fold_ptr, fold_list = _csr(slot, torch.arange(n_c), content_rows.numel())
    else:
        fold_ptr = fold_list = torch.zeros(0, dtype=torch.long)
    dev = lambda t: t.to(torch.int32).to(device)
    pad = lambda t: torch.cat((t, t.new_full((1,), -1)))  # a list array is never null, even when empty
    tensors = dict(content_order=dev(order), event_q=dev(eq), event_write=dev(ew), query_source=dev(qs),
                   query_history=dev(qh), content_bounds=dev(torch.tensor(tuple(plan.content_bounds))),
                   q_ptr=dev(q_ptr), q_list=dev(pad(q_list)), write_event=dev(write_event),
                   query_event=dev(query_event), history_ptr=dev(h_ptr), history_list=dev(pad(h_list)),
                   history_rows=dev(pad(h_rows)), fold_rows=dev(content_rows if shared else fold_ptr),
                   fold_ptr=dev(fold_ptr), fold_list=dev(fold_list))
    p = lambda name: tensors[name].data_ptr() if tensors[name].numel() else None
    cs = _lib.EventPlan(n_c, n_q, n_e, kernel, p("content_order"), p("event_q"), p("event_write"), p("query_source"),
                        p("query_history"), p("content_bounds"), len(plan.content_bounds) - 1, h_rows.numel(),
                        p("q_ptr"), p("q_list"), p("write_event"), p("query_event"), p("history_ptr"),
                        p("history_list"), p("history_rows"), content_rows.numel() if shared else 0,
                        p("fold_rows"), p("fold_ptr"), p("fold_list"))
    ep = EventPlan(device, kernel, n_h, n_c, n_q, n_e, tuple(plan.content_bounds), tuple(plan.event_bounds),
                   dev(hidden), dev(torch.nonzero(~read).flatten()), content_rows.numel() + n_q == n_h, tensors, cs)
    object.__setattr__(plan, "_cqgdn_event_plan", ep)
    return ep


def _columns(H, HK):
    """Column offsets of the fused projection: (C, z, a, b, P) with C = 2SK + SV the conv channels."""
    C = (2 * HK + H) * 128
    return C, C, C + H * 128, C + H * 128 + H, C + H * 128 + 2 * H


def _check_heads(heads, key_heads):
    ok = (4, 8, 16, 32)
    if heads not in ok or key_heads not in ok or heads % key_heads:
        raise ValueError(f"heads={heads}, key_heads={key_heads}: supported are 4, 8, 16, 32, key heads dividing heads")


class _LayerCore(torch.autograd.Function):
    @staticmethod
    def forward(ctx, proj, conv_weight, A_log, dt_bias, norm_weight, ep, H, HK, eps, scale):
        # proj may be a column slice of a wider tensor: every read uses its row stride PS
        S, n_h, PS = H * 128, proj.shape[0], proj.stride(0)
        C, zc, ac, bc, _ = _columns(H, HK)
        dev, st = proj.device, gdn._stream(proj.device)
        w = conv_weight.contiguous()
        alog, dtb, nw = A_log.float().contiguous(), dt_bias.float().contiguous(), norm_weight.float().contiguous()
        E = ep.n_events
        q, k, v = (torch.empty(E, H, 128, dtype=proj.dtype, device=dev) for _ in range(3))
        gb = torch.empty(2, E, H, dtype=torch.float32, device=dev)
        fws = torch.empty(_lib.lib().cqgdn_event_inputs_fwd_workspace_size(ep.n_content, H, HK), dtype=torch.uint8,
                          device=dev)
        a_ptr, b_ptr = proj[:, ac:].data_ptr(), proj[:, bc:].data_ptr()
        gdn.call("cqgdn_event_inputs_fwd", ctypes.byref(ep.cstruct), H, HK, gdn._ptr(proj), PS, a_ptr, PS, b_ptr, PS,
                 gdn._ptr(w), gdn._ptr(alog), gdn._ptr(dtb), gdn._ptr(q), gdn._ptr(k), gdn._ptr(v),
                 gdn._ptr(gb[0]), gdn._ptr(gb[1]), gdn._ptr(fws), fws.numel(), st)
        y, _, rws = gdn._forward(q[None], k[None], v[None], gb[0][None], gb[1][None], ep.event_bounds, True, scale,
                                 training=True)
        out = torch.empty(n_h, H, 128, dtype=proj.dtype, device=dev)
        rstd = torch.empty(n_h, H, dtype=torch.float32, device=dev)
        gdn.call("cqgdn_gated_norm_fwd", gdn._ptr(y), gdn._ptr(ep.hidden_index), n_h, H, proj[:, zc:].data_ptr(),
                 PS, gdn._ptr(nw), float(eps), gdn._ptr(out), gdn._ptr(rstd), st)
        ctx.save_for_backward(proj, w, alog, dtb, nw, q, k, v, gb, rws, y, rstd)
        ctx.ep, ctx.H, ctx.HK, ctx.scale = ep, H, HK, scale
        ctx.dtypes = (conv_weight.dtype, A_log.dtype, dt_bias.dtype, norm_weight.dtype)
        return out.reshape(n_h, S)

    @staticmethod
    def backward(ctx, dout):
        proj, w, alog, dtb, nw, q, k, v, gb, rws, y, rstd = ctx.saved_tensors
        ep, H, HK = ctx.ep, ctx.H, ctx.HK
        n_h, P, PS = proj.shape[0], proj.shape[1], proj.stride(0)
        C, zc, ac, bc, width = _columns(H, HK)
        dev, st = proj.device, gdn._stream(proj.device)
        # the gradient is a dense [rows, P] tensor (row stride P) whatever proj's stride
        full = ep.covers_all and P == width
        d_proj = (torch.empty if full else torch.zeros)(n_h, P, dtype=proj.dtype, device=dev)
        do = dout.contiguous()
        dy = torch.empty(ep.n_events, H, 128, dtype=proj.dtype, device=dev)
        dnw = torch.empty(128, dtype=torch.float32, device=dev)
        nws = torch.empty(max(_lib.lib().cqgdn_gated_norm_bwd_workspace_size(n_h, H), 16), dtype=torch.uint8,
                          device=dev)
        gdn.call("cqgdn_gated_norm_bwd", gdn._ptr(y), gdn._ptr(ep.hidden_index), gdn._ptr(ep.unread_events),
                 ep.unread_events.numel(), n_h, H, proj[:, zc:].data_ptr(), PS, gdn._ptr(nw), gdn._ptr(rstd),
                 gdn._ptr(do), gdn._ptr(dy), d_proj[:, zc:].data_ptr(), P, gdn._ptr(dnw), gdn._ptr(nws),
                 nws.numel(), st)
        dq, dk, dv, dg, db = gdn._backward(q[None], k[None], v[None], gb[0][None], gb[1][None], rws, dy,
                                           ep.event_bounds, True, ctx.scale)
        dw = torch.empty(w.shape, dtype=torch.float32, device=dev)
        dgate = torch.empty(2 * H, dtype=torch.float32, device=dev)
        ews = torch.empty(_lib.lib().cqgdn_event_inputs_bwd_workspace_size(ctypes.byref(ep.cstruct), H, HK),
                          dtype=torch.uint8, device=dev)
        gdn.call("cqgdn_event_inputs_bwd", ctypes.byref(ep.cstruct), H, HK, gdn._ptr(proj), PS,
                 proj[:, ac:].data_ptr(), PS, proj[:, bc:].data_ptr(), PS, gdn._ptr(w), gdn._ptr(alog),
                 gdn._ptr(dtb), gdn._ptr(dq), gdn._ptr(dk), gdn._ptr(dv), gdn._ptr(dg), gdn._ptr(db),
                 gdn._ptr(d_proj), P, d_proj[:, ac:].data_ptr(), P, d_proj[:, bc:].data_ptr(), P,
                 gdn._ptr(dw), gdn._ptr(dgate), gdn._ptr(ews), ews.numel(), st)
        cw, ca, cd, cn = ctx.dtypes
        return d_proj, dw.to(cw), dgate[:H].to(ca), dgate[H:].to(cd), dnw.to(cn), None, None, None, None, None


def layer_core(proj, conv_weight, A_log, dt_bias, norm_weight, plan, *, heads, key_heads=None, eps=1e-6,
               scale=None):
    """GatedDelta between its projections: proj [rows, 2SK + 2SV + 2H] bf16 (q|k|v, z, a, b columns
    of ``in_proj_all``; SK = key_heads * 128, SV = heads * 128), conv_weight [2SK + SV, K] bf16,
    A_log / dt_bias [H], norm_weight [128]; returns the gated-norm rows [rows, SV] that feed
    ``out_proj`` (models/backbone_qwen35.py:158-246, training path).  ``key_heads`` (the
    reference's linear_heads per rank) defaults to ``heads``."""
    HK = heads if key_heads is None else int(key_heads)
    _check_heads(heads, HK)
    C, _, _, _, width = _columns(heads, HK)
    if proj.dim() != 2 or proj.shape[1] != width or proj.stride(1) != 1:
        raise ValueError("proj must be [rows, (2*key_heads + 2*heads)*128 + 2*heads] with unit column stride")
    if proj.dtype != torch.bfloat16 or conv_weight.dtype != torch.bfloat16:
        raise NotImplementedError("the fused layer kernels compute on bf16 projections and conv weights")
    if conv_weight.shape[0] != C or A_log.shape != (heads,) or dt_bias.shape != (heads,) or \
            norm_weight.shape != (128,):
        raise ValueError("parameter shapes do not match the head counts")
    gdn._require_gpu(proj, conv_weight, A_log, dt_bias, norm_weight)
    if proj.stride(0) < proj.shape[1] or proj.stride(0) % 8 or proj.data_ptr() % 16:
        proj = proj.contiguous()  # the kernels read rows proj.stride(0) apart with 16-byte loads
    ep = event_plan(plan, conv_weight.shape[1], proj.device)
    if ep.n_hidden != proj.shape[0]:
        raise ValueError("proj rows do not match the plan's hidden rows")
    return _LayerCore.apply(proj, conv_weight, A_log, dt_bias, norm_weight, ep, heads, HK, eps,
                            128 ** -0.5 if scale is None else float(scale))


@torch.no_grad()
def layer_prefill(proj, conv_weight, A_log, dt_bias, norm_weight, plan, *, heads, key_heads=None, eps=1e-6,
                  scale=None):
    """Inference prefill of the layer with the cache a decoder continues from
    (models/backbone_qwen35.py:163-211 with ``cache``): the event inputs as in training, the
    precise forward with each document's final state, the gated norm with the output gather.

    Heads and columns as in ``layer_core``.  Returns ``(out [rows, SV], cache)``: ``cache["state"]``
    fp32 [n_docs, H, V, K] value-first (the decode layout) and ``cache["conv"]`` bf16 [1, K-1, C],
    the raw q|k|v rows of the K-1 content rows before the last one, zero-filled in front, as the
    reference keeps them (its last content row is the uncommitted target, models/decoding.py:117-121)."""
    HK = heads if key_heads is None else int(key_heads)
    _check_heads(heads, HK)
    S = heads * 128
    C, zc, ac, bc, width = _columns(heads, HK)
    if proj.dim() != 2 or proj.shape[1] != width or proj.dtype != torch.bfloat16:
        raise ValueError("proj must be bf16 [rows, (2*key_heads + 2*heads)*128 + 2*heads]")
    gdn._require_gpu(proj, conv_weight)
    proj = proj.contiguous()
    K = conv_weight.shape[1]
    ep = event_plan(plan, K, proj.device)
    dev, st, P, n_h, E = proj.device, gdn._stream(proj.device), proj.shape[1], proj.shape[0], ep.n_events
    w = conv_weight.contiguous()
    alog, dtb, nw = A_log.float().contiguous(), dt_bias.float().contiguous(), norm_weight.float().contiguous()
    q, k, v = (torch.empty(E, heads, 128, dtype=proj.dtype, device=dev) for _ in range(3))
    gb = torch.empty(2, E, heads, dtype=torch.float32, device=dev)
    fws = torch.empty(_lib.lib().cqgdn_event_inputs_fwd_workspace_size(ep.n_content, heads, HK),
                      dtype=torch.uint8, device=dev)
    gdn.call("cqgdn_event_inputs_fwd", ctypes.byref(ep.cstruct), heads, HK, gdn._ptr(proj), P,
             proj[:, ac:].data_ptr(), P, proj[:, bc:].data_ptr(), P, gdn._ptr(w), gdn._ptr(alog),
             gdn._ptr(dtb), gdn._ptr(q), gdn._ptr(k), gdn._ptr(v), gdn._ptr(gb[0]), gdn._ptr(gb[1]), gdn._ptr(fws),
             fws.numel(), st)
    y, state, _ = gdn._forward(q[None], k[None], v[None], gb[0][None], gb[1][None], ep.event_bounds, True,
                               128 ** -0.5 if scale is None else float(scale), training=False, want_state=True,
                               precise=True)
    out = torch.empty(n_h, heads, 128, dtype=proj.dtype, device=dev)
    rstd = torch.empty(n_h, heads, dtype=torch.float32, device=dev)
    gdn.call("cqgdn_gated_norm_fwd", gdn._ptr(y), gdn._ptr(ep.hidden_index), n_h, heads, proj[:, zc:].data_ptr(),
             P, gdn._ptr(nw), float(eps), gdn._ptr(out), gdn._ptr(rstd), st)
    count = K - 1
    history = proj.new_zeros(1, count, C)
    order = ep.tensors["content_order"]
    tail = order[max(0, ep.n_content - 1 - count):max(ep.n_content - 1, 0)].long()
    if tail.numel():
        history[0, count - tail.numel():] = proj.index_select(0, tail)[:, :C]
    return out.reshape(n_h, S), {"state": state.transpose(-1, -2).contiguous(), "conv": history}


@torch.no_grad()
def layer_decode_step(proj, conv_weight, A_log, dt_bias, norm_weight, cache, *, heads, key_heads=None, eps=1e-6,
                      scale=None):
    """One decode step (models/decoding.py:16-78 between the projection and out_proj) for N
    sequences: proj [N, 2, P] bf16 (row 0 the sampled content token, row 1 the text-mask query;
    [2, P] for one sequence; heads and columns as in ``layer_core``); ``cache["conv"]`` bf16
    [N, K-1, C] and ``cache["state"]`` fp32 [N, H, V, K] are updated in place.  Returns the
    gated-norm rows [N, 2, SV] ([2, SV])."""
    # the contract checks (shapes, dtypes, contiguity, device) run inside the operator, before the launch
    single = proj.dim() == 2
    gdn.CALLS["cqgdn_layer_decode_step"] += 1
    out = _lib.ops().layer_decode_step(proj[None] if single else proj, conv_weight, A_log, dt_bias, norm_weight,
                                       cache["conv"], cache["state"], heads, heads if key_heads is None else key_heads,
                                       eps, 128 ** -0.5 if scale is None else scale)
    return out[0] if single else out
