"""CPU oracle for the gated delta-rule (GDN) recurrence.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker (or, for ``cpu_baseline``, as the CPU path that is timed).  The product
path (``cq-pretrain_amd/cqgdn``) never imports it: it runs the HIP kernels of
``libcqgdn.so`` or raises.

Everything here is plain PyTorch on the CPU (float64 by default), restating the
reference's own algorithms:

* ``l2norm``            - ``assets/Qwen3.5-0.8B/reference_modeling_qwen3_5.py:280-283``
* ``recurrent_delta``   - ``models/backbone_qwen35.py:56-72`` and
                          ``scripts/validation/delta64_probe.py:102-118`` (per-event loop,
                          state reset at every document start)
* ``chunk_delta``       - ``reference_modeling_qwen3_5.py:287-420`` (chunked WY/UT form,
                          chunk 64), applied per document of ``bounds``; the intermediates
                          follow ``scripts/validation/delta_ascendc_diagnose.py:23-37``
* ``chunk_delta_backward`` - the analytic backward of ``chunk_delta`` split the way the
                          HIP kernels split it (local dv / state-gradient scan / dq,dk,dw,dg /
                          WY backward); the reference's own backward is the op chain of
                          ``ops/gated_delta_net.py:188-214``
* ``decode_step``       - ``models/decoding.py:71-77`` with the value-first state and
                          in-place contract of ``ops/gated_delta_net.py:314-352``
* ``error_stats``       - ``scripts/validation/delta64_probe.py:90-99``
* ``causal_conv1d``     - the GatedDelta layer's short conv, the CPU form of
                          ``models/backbone_qwen35.py:81-98`` (``F.conv1d`` with padding K-1 per
                          document, optional SiLU) behind ``ops/gated_delta_net.py:252-289``
* ``gated_rms_norm``    - the layer's gated norm, ``models/backbone_qwen35.py:107-114`` behind
                          ``ops/gated_delta_net.py:67-74``
* ``layer_decode_step`` - one decode step of the layer between its projections,
                          ``models/decoding.py:16-78`` (CPU path), composed of the pieces above

How each function is pinned (tests/test_oracle.py): closed forms on tiny inputs
(one event, orthonormal keys, pure decay), chunked == per-event recurrence to
1e-10 in float64, the UT inverse against ``torch.linalg.solve_triangular``,
autograd ``gradcheck`` of the recurrence against finite differences, the manual
backward against autograd of the recurrence, document isolation and the
read-only-event invariants of ``tests/test_qwen35_cq.py:71-89``.
"""

from __future__ import annotations

import torch

EPS = 1e-6
CHUNK = 64


def l2norm(x, eps=EPS):
    """x * rsqrt(sum(x^2) + eps) over the last dim (reference_modeling_qwen3_5.py:280-283)."""
    return x * torch.rsqrt(x.square().sum(-1, keepdim=True) + eps)


def _bounds(bounds, t):
    if bounds is None:
        return (0, t)
    return tuple(int(b) for b in bounds)


def recurrent_delta(q, k, v, g, beta, bounds=None, *, normalize=True, scale=None,
                    initial_state=None, output_final_state=False):
    """Per-event gated delta rule (models/backbone_qwen35.py:56-72).

    q, k: [B,T,H,K]; v: [B,T,H,V]; g, beta: [B,T,H].  ``bounds`` are document
    boundaries ``(0, ..., T)`` (B must then be 1); the state resets to zero (or to
    ``initial_state[doc]``) at each document start.  Returns o [B,T,H,V] and, if
    asked, the final state per document [N,H,K,V] (key-first).
    """
    scale = q.shape[-1] ** -0.5 if scale is None else scale
    if normalize:
        q, k = l2norm(q), l2norm(k)
    q = q * scale
    bounds = _bounds(bounds, q.shape[1])
    outputs, states = [], []
    for d, (begin, end) in enumerate(zip(bounds, bounds[1:])):
        if initial_state is None:
            state = q.new_zeros(q.shape[0], q.shape[2], q.shape[3], v.shape[3])
        else:
            state = initial_state[d:d + 1].to(q.dtype).expand(q.shape[0], -1, -1, -1)
        for i in range(begin, end):
            state = state * g[:, i].exp()[..., None, None]
            residual = v[:, i] - (state * k[:, i, :, :, None]).sum(-2)
            state = state + k[:, i, :, :, None] * (residual * beta[:, i, :, None])[..., None, :]
            outputs.append((state * q[:, i, :, :, None]).sum(-2))
        states.append(state)
    out = torch.stack(outputs, dim=1) if outputs else v.new_zeros(v.shape)
    if output_final_state:
        return out, torch.cat(states) if states else None
    return out


def _chunk_spans(begin, end, chunk):
    return [(a, min(a + chunk, end)) for a in range(begin, end, chunk)]


def chunk_delta(q, k, v, g, beta, bounds=None, *, chunk=CHUNK, normalize=True, scale=None,
                initial_state=None, output_final_state=False, return_intermediates=False):
    """Chunked WY/UT form of the gated delta rule (reference_modeling_qwen3_5.py:287-420).

    Same contract as ``recurrent_delta`` with B == 1.  Chunks never cross a
    document boundary; a document's last chunk holds its tail (the reference pads
    the tail with zero k/v/beta/g rows, which is the same computation).

    With ``return_intermediates`` the per-chunk tensors the HIP kernels produce are
    returned in a dict, each a list over chunks (in the chunk-table order of
    ``chunk_spans``) of tensors shaped per head:
      gcum [H,C], A [H,C,C] (strict lower), T [H,C,C] = (I+A)^-1, W [H,C,K],
      U [H,C,V], h [H,K,V] (state entering the chunk), vn [H,C,V],
    plus the normalized inputs qn, kn [1,T,H,K].
    """
    if q.shape[0] != 1:
        raise ValueError("chunk_delta expects batch 1 (packed documents)")
    scale = q.shape[-1] ** -0.5 if scale is None else scale
    if normalize:
        q, k = l2norm(q), l2norm(k)
    bounds = _bounds(bounds, q.shape[1])
    qh, kh, vh = (x[0].transpose(0, 1) for x in (q, k, v))  # [H,T,D]
    gh, bh = g[0].transpose(0, 1), beta[0].transpose(0, 1)  # [H,T]
    H, K, V = qh.shape[0], qh.shape[2], vh.shape[2]
    out = torch.zeros_like(vh)
    inter = dict(gcum=[], A=[], T=[], W=[], U=[], h=[], vn=[], spans=[])
    finals = []
    for d, (begin, end) in enumerate(zip(bounds, bounds[1:])):
        S = qh.new_zeros(H, K, V) if initial_state is None else initial_state[d].to(qh.dtype)
        for a, b in _chunk_spans(begin, end, chunk):
            n = b - a
            qc, kc, vc, gc, bc = qh[:, a:b], kh[:, a:b], vh[:, a:b], gh[:, a:b], bh[:, a:b]
            G = gc.cumsum(-1)
            incl = torch.ones(n, n, dtype=torch.bool).tril()
            strict = torch.ones(n, n, dtype=torch.bool).tril(-1)
            Gam = (G[:, :, None] - G[:, None, :]).masked_fill(~incl, float("-inf")).exp()
            A = (bc[:, :, None] * (kc @ kc.transpose(-1, -2)) * Gam).masked_fill(~strict, 0)
            eye = torch.eye(n, dtype=qh.dtype).expand(H, n, n)
            T = torch.linalg.solve_triangular(A + eye, eye, upper=False, unitriangular=True)
            gam = G.exp()
            W = T @ ((bc * gam)[..., None] * kc)
            U = T @ (bc[..., None] * vc)
            vn = U - W @ S
            P = (qc @ kc.transpose(-1, -2)) * Gam
            out[:, a:b] = scale * ((gam[..., None] * qc) @ S + P @ vn)
            gl = G[:, -1:]
            if return_intermediates:
                for key, val in zip(("gcum", "A", "T", "W", "U", "h", "vn"), (G, A, T, W, U, S, vn)):
                    inter[key].append(val)
                inter["spans"].append((a, b))
            S = gl.exp()[..., None] * S + ((gl - G).exp()[..., None] * kc).transpose(-1, -2) @ vn
        finals.append(S)
    o = out.transpose(0, 1)[None]
    result = [o]
    if output_final_state:
        result.append(torch.stack(finals) if finals else None)
    if return_intermediates:
        inter["qn"], inter["kn"] = q, k
        result.append(inter)
    return result[0] if len(result) == 1 else tuple(result)


def chunk_spans(bounds, chunk=CHUNK):
    """Chunk table: (start, end) of every chunk, documents in order (ops/gated_delta_net.py:90-99)."""
    return [s for a, b in zip(bounds, bounds[1:]) for s in _chunk_spans(a, b, chunk)]


def chunk_delta_backward(q, k, v, g, beta, do, bounds=None, *, chunk=CHUNK, normalize=True,
                         scale=None, return_intermediates=False):
    """Analytic backward of ``chunk_delta`` in the decomposition the HIP kernels use.

    Per chunk (C events, state S_c entering it, dS_{c+1} the gradient of the state
    leaving it), with Gam_ij = exp(G_i - G_j) on i >= j, gam = exp(G),
    kdec_i = exp(G_last - G_i), P = (Qn Kn^T) * Gam:

      local:   dv_local = scale * P^T dO ;  X = scale * (gam*Qn)^T dO
      scan:    dVn = dv_local + kdec * (Kn dS_{c+1}) ;
               dS_c = exp(G_last) dS_{c+1} + X - W^T dVn
      dq/dk/dw/dg:  dQn = scale*gam*(dO S_c^T) + (scale*dP*Gam) Kn, dP = dO Vn^T
               dKn = (scale*dP*Gam)^T Qn + kdec*(Vn dS_{c+1}^T);  dW = -dVn S_c^T
      WY:      dT = dW (beta*gam*Kn)^T + dVn (beta*V)^T ;  dA = -(T^T dT T^T) strict lower
               dKn += beta*(dA*Gam) Kn + (dA*Gam)^T (beta*Kn) + beta*gam*(T^T dW)
               dV = beta*(T^T dVn);  dbeta, dG from every beta/G use;  dg = reverse cumsum dG
    then the l2norm backward dq = rq*(dQn - Qn (Qn.dQn)).  Returns (dq, dk, dv, dg, dbeta)
    shaped like the inputs, and optionally a dict of per-chunk intermediates
    (dv_local, X, dh = dS_{c+1}, dVn).
    """
    scale = q.shape[-1] ** -0.5 if scale is None else scale
    _, _, inter = chunk_delta(q, k, v, g, beta, bounds, chunk=chunk, normalize=normalize, scale=scale,
                              output_final_state=True, return_intermediates=True)
    qn, kn = inter["qn"], inter["kn"]
    qh, kh, vh, doh = (x[0].transpose(0, 1) for x in (qn, kn, v, do))
    gh, bh = g[0].transpose(0, 1), beta[0].transpose(0, 1)
    H, K, V = qh.shape[0], qh.shape[2], vh.shape[2]
    dqh, dkh, dvh = torch.zeros_like(qh), torch.zeros_like(kh), torch.zeros_like(vh)
    dgh, dbh = torch.zeros_like(gh), torch.zeros_like(bh)
    bounds = _bounds(bounds, q.shape[1])
    spans = inter["spans"]
    index = {s: i for i, s in enumerate(spans)}
    binter = dict(dv_local=[None] * len(spans), X=[None] * len(spans), dh=[None] * len(spans),
                  dVn=[None] * len(spans))
    for begin, end in zip(bounds, bounds[1:]):
        dS = qh.new_zeros(H, K, V)
        for a, b in reversed(_chunk_spans(begin, end, chunk)):
            c = index[(a, b)]
            n = b - a
            G, T, W, S, vn = (inter[key][c] for key in ("gcum", "T", "W", "h", "vn"))
            A = inter["A"][c]
            qc, kc, vc, doc, bc = qh[:, a:b], kh[:, a:b], vh[:, a:b], doh[:, a:b], bh[:, a:b]
            incl = torch.ones(n, n, dtype=torch.bool).tril()
            strict = torch.ones(n, n, dtype=torch.bool).tril(-1)
            Gam = (G[:, :, None] - G[:, None, :]).masked_fill(~incl, float("-inf")).exp()
            gam = G.exp()
            gl = G[:, -1]
            kdec = (gl[:, None] - G).exp()
            P = (qc @ kc.transpose(-1, -2)) * Gam
            # local stage
            dv_local = scale * P.transpose(-1, -2) @ doc
            X = scale * (gam[..., None] * qc).transpose(-1, -2) @ doc
            # state-gradient scan stage
            dh = dS
            dVn = dv_local + kdec[..., None] * (kc @ dh)
            dS = gl.exp()[:, None, None] * dh + X - W.transpose(-1, -2) @ dVn
            # dq / dk / dw / dg stage
            dP = doc @ vn.transpose(-1, -2)
            dPm = scale * dP * Gam
            dQ_inter = scale * gam[..., None] * (doc @ S.transpose(-1, -2))
            dQ = dQ_inter + dPm @ kc
            dK_state = kdec[..., None] * (vn @ dh.transpose(-1, -2))
            dK = dPm.transpose(-1, -2) @ qc + dK_state
            dW = -dVn @ S.transpose(-1, -2)
            dG = (qc * dQ_inter).sum(-1)
            E = scale * dP * P
            dG = dG + E.sum(-1) - E.sum(-2)
            e = (kc * dK_state).sum(-1)
            dG = dG - e
            dG[:, -1] += gl.exp() * (S * dh).sum((-1, -2)) + e.sum(-1)
            # WY stage
            kbg = (bc * gam)[..., None] * kc
            vb = bc[..., None] * vc
            dT = dW @ kbg.transpose(-1, -2) + dVn @ vb.transpose(-1, -2)
            Tt = T.transpose(-1, -2)
            dA = (-(Tt @ dT @ Tt)).masked_fill(~strict, 0)
            dM = dA * Gam
            KK = kc @ kc.transpose(-1, -2)
            dK = dK + bc[..., None] * (dM @ kc) + dM.transpose(-1, -2) @ (bc[..., None] * kc)
            dB = (dM * KK).sum(-1)
            E2 = dA * A
            dG = dG + E2.sum(-1) - E2.sum(-2)
            TdW = Tt @ dW
            kTdW = (kc * TdW).sum(-1)
            dK = dK + (bc * gam)[..., None] * TdW
            dB = dB + gam * kTdW
            dG = dG + bc * gam * kTdW
            TdU = Tt @ dVn
            dvh[:, a:b] = bc[..., None] * TdU
            dB = dB + (vc * TdU).sum(-1)
            dgh[:, a:b] = dG.flip(-1).cumsum(-1).flip(-1)
            dbh[:, a:b] = dB
            dqh[:, a:b] = dQ
            dkh[:, a:b] = dK
            if return_intermediates:
                binter["dv_local"][c], binter["X"][c] = dv_local, X
                binter["dh"][c], binter["dVn"][c] = dh, dVn
    dq_n, dk_n = dqh.transpose(0, 1)[None], dkh.transpose(0, 1)[None]
    if normalize:
        rq = torch.rsqrt(q.square().sum(-1, keepdim=True) + EPS)
        rk = torch.rsqrt(k.square().sum(-1, keepdim=True) + EPS)
        dq = rq * (dq_n - qn * (qn * dq_n).sum(-1, keepdim=True))
        dk = rk * (dk_n - kn * (kn * dk_n).sum(-1, keepdim=True))
    else:
        dq, dk = dq_n, dk_n
    grads = (dq, dk, dvh.transpose(0, 1)[None], dgh.transpose(0, 1)[None], dbh.transpose(0, 1)[None])
    if return_intermediates:
        return grads, binter
    return grads


def decode_step(q, k, v, g, beta, state, scale=None):
    """Recurrent GDN step(s) on a value-first state, in place (models/decoding.py:71-77).

    Follows the contract of ``ops/gated_delta_net.py:314-352``: q and k are already
    l2-normalized; ``state`` is [N,H,V,K] float (value-first) and is updated in
    place; q,k,v are [N,E,H,D] with E events applied in order to each of the N
    independent sequences; g, beta are [N,E,H].  Returns o [N,E,H,V] in float.
    """
    scale = q.shape[-1] ** -0.5 if scale is None else scale
    outs = []
    for e in range(q.shape[1]):
        qe, ke, ve = (x[:, e].to(state.dtype) for x in (q, k, v))
        ge, be = g[:, e].to(state.dtype), beta[:, e].to(state.dtype)
        state.mul_(ge.exp()[..., None, None])
        residual = ve - torch.matmul(state, ke[..., None]).squeeze(-1)
        state.add_((residual * be[..., None])[..., None] * ke[..., None, :])
        outs.append(scale * torch.matmul(state, qe[..., None]).squeeze(-1))
    return torch.stack(outs, dim=1)


def chunk_local_cumsum(g, bounds=None, chunk=CHUNK, reverse=False):
    """Cumsum of g [B,T,H] within every chunk of every document (ops/gated_delta_net.py:77-87)."""
    out = torch.empty_like(g)
    for a, b in chunk_spans(_bounds(bounds, g.shape[1]), chunk):
        seg = g[:, a:b]
        out[:, a:b] = seg.flip(1).cumsum(1).flip(1) if reverse else seg.cumsum(1)
    return out


def causal_conv1d(x, weight, bounds=None, activation=True):
    """Depthwise causal conv1d over packed documents (models/backbone_qwen35.py:81-98).

    x: [1,T,C] (or [B,T,C] with ``bounds`` None: one document per row); weight: [C,K].
    Row t of a document sees rows t-K+1 .. t of the same document only.
    """
    weight = weight.to(x.dtype)
    bounds = _bounds(bounds, x.shape[1]) if bounds is not None else None
    spans = list(zip(bounds, bounds[1:])) if bounds is not None else [(0, x.shape[1])]
    parts = []
    for a, b in spans:
        seg = x[:, a:b].transpose(1, 2)
        y = torch.nn.functional.conv1d(seg, weight[:, None], padding=weight.shape[1] - 1, groups=x.shape[-1])
        parts.append(y[..., : b - a].transpose(1, 2))
    y = torch.cat(parts, dim=1) if parts else x[:, :0]
    return torch.nn.functional.silu(y) if activation else y


def gated_rms_norm(y, z, weight, eps=1e-6):
    """RMSNorm over the last dimension, times weight and silu(z): the CPU form of the layer's
    gated norm (models/backbone_qwen35.py:107-114), behind gated_norm (ops/gated_delta_net.py:67-74)."""
    y, z = y.double(), z.double()
    normalized = y * torch.rsqrt(y.square().mean(-1, keepdim=True) + eps)
    return normalized * weight.double() * torch.nn.functional.silu(z)


def layer_decode_step(raw, z, a, b, conv_weight, A_log, dt_bias, norm_weight, history, state, eps=1e-6):
    """One decode step of the GatedDelta layer between its projections, the CPU path of
    models/decoding.py:16-78, in float64 for N sequences.

    raw [N, 2, C] (row 0 the sampled content token C, row 1 the text-mask query Q; channels
    q | k | v, C = 2 SK + SV with SK = HK * 128 key channels and SV = H * 128 value channels), z
    [N, 2, H, D], a, b [N, 2, H]; history [N, K-1, C]; state [N, H, V, K] value-first.
    C's conv reads the history, which then shifts in C's raw row; Q's query conv reads the
    shifted history; with HK < H key heads, q and k repeat each key head for H // HK value
    heads (models/decoding.py:52-53); the recurrence applies C and then the read-only Q.
    Returns (out [N, 2, H, D], history, state) without touching the inputs.
    """
    n, H, K = raw.shape[0], A_log.shape[0], conv_weight.shape[1]
    SV = H * 128
    SK = (raw.shape[-1] - SV) // 2
    silu, w, x = torch.nn.functional.silu, conv_weight.double(), raw.double()
    hist = history.double()
    conv = silu(x[:, 0] * w[:, -1] + sum(hist[:, j] * w[:, j] for j in range(K - 1)))
    hist = torch.cat((hist[:, 1:], x[:, :1]), dim=1)
    query = silu(x[:, 1, :SK] * w[:SK, -1] + sum(hist[:, j, :SK] * w[:SK, j] for j in range(K - 1)))
    cq, k, v = conv.split((SK, SK, SV), -1)
    zero_k, zero_v = torch.zeros_like(k), torch.zeros_like(v)
    rep = H // (SK // 128)
    q = torch.stack((cq, query), 1).reshape(n, 2, SK // 128, 128).repeat_interleave(rep, dim=2)
    k = torch.stack((k, zero_k), 1).reshape(n, 2, SK // 128, 128).repeat_interleave(rep, dim=2)
    v = torch.stack((v, zero_v), 1).reshape(n, 2, H, 128)
    g = -A_log.double().exp() * torch.nn.functional.softplus(a[:, 0].double() + dt_bias.double())
    beta = b[:, 0].double().sigmoid()
    g, beta = torch.stack((g, torch.zeros_like(g)), 1), torch.stack((beta, torch.zeros_like(beta)), 1)
    st = state.double().clone()
    y = decode_step(l2norm(q), l2norm(k), v, g, beta, st)
    return gated_rms_norm(y, z, norm_weight, eps), hist, st


def error_stats(actual, expected, tolerance=0.035):
    """Relative-L2 error with a max-abs escape (scripts/validation/delta64_probe.py:90-99)."""
    a, b = actual.detach().cpu().double(), expected.detach().cpu().double()
    actual_finite, expected_finite = bool(torch.isfinite(a).all()), bool(torch.isfinite(b).all())
    delta = a - b
    relative = float(delta.norm() / b.norm().clamp_min(1e-12))
    absolute = float(delta.abs().max()) if delta.numel() else 0.0
    return dict(relative_l2=relative, max_abs=absolute, tolerance=tolerance,
                actual_finite=actual_finite, expected_finite=expected_finite,
                passed=actual_finite and expected_finite and (relative <= tolerance or absolute <= 2e-7))


def make_inputs(T, H=16, D=128, *, seed=0, dtype=torch.bfloat16, readonly=None, generator_dtype=torch.float32):
    """Seeded synthetic GDN inputs with the distributions of the benchmark configs.

    q,k,v ~ N(0,1) in ``dtype``; beta = sigmoid(N(0,1)); g = -softplus(N(0,1)); both
    float32 [1,T,H].  ``readonly`` is a bool mask [T] of read-only (query) events,
    which carry a real q but k = v = 0 and g = beta = 0
    (models/backbone_qwen35.py:184-194).
    """
    gen = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(1, T, H, D, generator=gen, dtype=generator_dtype).to(dtype) for _ in range(3))
    beta = torch.randn(1, T, H, generator=gen, dtype=generator_dtype).sigmoid()
    g = -torch.nn.functional.softplus(torch.randn(1, T, H, generator=gen, dtype=generator_dtype))
    if readonly is not None:
        m = torch.as_tensor(readonly, dtype=torch.bool)
        k[:, m] = 0
        v[:, m] = 0
        g[:, m] = 0
        beta[:, m] = 0
    return q, k, v, g.float(), beta.float()
