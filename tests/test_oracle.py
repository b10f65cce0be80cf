"""Pins the CPU oracle (oracle/gdn_oracle.py) on the CPU, before it is trusted as the checker.

Each function is tied to something that fixes it independently of its own code:
golden vectors written by plain-Python arithmetic (tests/golden/), closed forms
on tiny inputs (one event, orthonormal keys, pure decay), the per-event
recurrence (chunked == recurrent to 1e-10 in float64), library routines
(``torch.linalg.inv`` for the UT inverse, autograd and finite differences for
the gradients) and the exact read-only / document invariants the reference
tests (tests/test_qwen35_cq.py:71-89, tests/test_document_packing.py:180-200).
The last tests plant mistakes in the oracle and check that these pins catch them.
"""

import json
import math
from pathlib import Path

import pytest
import torch

from oracle import gdn_oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden"
F64 = torch.float64


def rand_inputs(T, H, D, seed, dtype=F64):
    gen = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(1, T, H, D, generator=gen, dtype=dtype) for _ in range(3))
    beta = torch.randn(1, T, H, generator=gen, dtype=dtype).sigmoid()
    g = -torch.nn.functional.softplus(torch.randn(1, T, H, generator=gen, dtype=dtype))
    return q, k, v, g, beta


# ---------------------------------------------------------------- golden vectors
def test_recurrence_matches_plain_python_golden():
    gv = json.loads((GOLDEN / "recurrence_d8.json").read_text())
    q, k, v = (torch.tensor(gv[n], dtype=F64)[None] for n in ("q", "k", "v"))
    g, beta = (torch.tensor(gv[n], dtype=F64)[None] for n in ("g", "beta"))
    o_ref, s_ref = torch.tensor(gv["o"], dtype=F64)[None], torch.tensor(gv["final_state"], dtype=F64)
    bounds = tuple(gv["bounds"])
    o, s = O.recurrent_delta(q, k, v, g, beta, bounds, output_final_state=True)
    torch.testing.assert_close(o, o_ref, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(s, s_ref, rtol=1e-12, atol=1e-12)
    oc, sc = O.chunk_delta(q, k, v, g, beta, bounds, output_final_state=True)
    torch.testing.assert_close(oc, o_ref, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(sc, s_ref, rtol=1e-10, atol=1e-10)


def test_decode_step_matches_plain_python_golden():
    gv = json.loads((GOLDEN / "decode_d8.json").read_text())
    q, k, v, g, beta = (torch.tensor(gv[n], dtype=F64) for n in ("q", "k", "v", "g", "beta"))
    state = torch.tensor(gv["state_in"], dtype=F64)
    out = O.decode_step(q, k, v, g, beta, state)
    torch.testing.assert_close(out, torch.tensor(gv["out"], dtype=F64), rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(state, torch.tensor(gv["state_out"], dtype=F64), rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------- closed forms
def test_l2norm_closed_form():
    x = torch.tensor([[3.0, 4.0], [0.0, 0.0]], dtype=F64)
    y = O.l2norm(x)
    torch.testing.assert_close(y[0], torch.tensor([3.0, 4.0], dtype=F64) / math.sqrt(25 + 1e-6))
    assert torch.equal(y[1], torch.zeros(2, dtype=F64))  # zero rows stay zero (read-only k)


def test_single_event_closed_form():
    # one event from S = 0: S = beta k^ v^T, o = d^-1/2 (q^.k^) beta v
    q, k, v, g, beta = rand_inputs(1, 3, 16, seed=1)
    o, s = O.recurrent_delta(q, k, v, g, beta, output_final_state=True)
    qn, kn = q / q.norm(dim=-1, keepdim=True), k / k.norm(dim=-1, keepdim=True)
    dot = (qn * kn).sum(-1, keepdim=True)
    torch.testing.assert_close(o, 16 ** -0.5 * beta[..., None] * dot * v, rtol=1e-6, atol=1e-9)
    torch.testing.assert_close(s[0], beta[0, 0, :, None, None] * kn[0, 0, :, :, None] * v[0, 0, :, None, :],
                               rtol=1e-6, atol=1e-9)


def test_orthonormal_keys_store_and_retrieve():
    # beta = 1, g = 0, keys = basis vectors: S = sum_i e_i v_i^T, so reading with q = e_i returns v_i * d^-1/2
    D, n = 8, 5
    eye = torch.eye(D, dtype=F64)
    k = eye[:n][None, :, None]  # [1,n,1,D]
    v = torch.randn(1, n, 1, D, dtype=F64, generator=torch.Generator().manual_seed(2))
    q = torch.cat([k, k], dim=1)  # read each key after all writes (2n events, second half read-only)
    kk = torch.cat([k, torch.zeros_like(k)], dim=1)
    vv = torch.cat([v, torch.zeros_like(v)], dim=1)
    g = torch.zeros(1, 2 * n, 1, dtype=F64)
    beta = torch.cat([torch.ones(1, n, 1, dtype=F64), torch.zeros(1, n, 1, dtype=F64)], dim=1)
    for fn in (O.recurrent_delta, O.chunk_delta):
        o = fn(q, kk, vv, g, beta)
        torch.testing.assert_close(o[:, n:], v * D ** -0.5, rtol=1e-6, atol=1e-9)


def test_overwrite_with_beta_one_replaces_value():
    # the delta rule with beta = 1 on a unit key replaces the stored value exactly (keys given already
    # normalized: the 1e-6 inside l2norm would leave |k| = 1 - 5e-7)
    D = 8
    e0 = torch.eye(D, dtype=F64)[0]
    k = e0.expand(1, 3, 1, D).clone()
    v = torch.randn(1, 3, 1, D, dtype=F64, generator=torch.Generator().manual_seed(3))
    q = k.clone()
    g = torch.zeros(1, 3, 1, dtype=F64)
    beta = torch.ones(1, 3, 1, dtype=F64)
    _, s = O.recurrent_delta(q, k, v, g, beta, normalize=False, output_final_state=True)
    expected = torch.zeros(D, D, dtype=F64)
    expected[0] = v[0, -1, 0]
    torch.testing.assert_close(s[0, 0], expected, rtol=1e-14, atol=1e-14)


def test_pure_decay_of_initial_state():
    # beta = 0: S_t = exp(sum g) S_0 and o_t = d^-1/2 exp(cumsum g)_t S_0^T q^_t
    T, H, D = 70, 2, 16
    q, k, v, g, _ = rand_inputs(T, H, D, seed=4)
    beta = torch.zeros(1, T, H, dtype=F64)
    s0 = torch.randn(1, H, D, D, dtype=F64, generator=torch.Generator().manual_seed(5))
    qn = q / torch.sqrt(q.square().sum(-1, keepdim=True) + 1e-6)
    decay = g.cumsum(1).exp()  # [1,T,H]
    expected = D ** -0.5 * decay[..., None] * torch.einsum("hkv,thk->thv", s0[0], qn[0])[None]
    for fn in (O.recurrent_delta, O.chunk_delta):
        o, s = fn(q, k, v, g, beta, initial_state=s0, output_final_state=True)
        torch.testing.assert_close(o, expected, rtol=1e-10, atol=1e-12)
        torch.testing.assert_close(s, decay[0, -1][None, :, None, None] * s0, rtol=1e-10, atol=1e-12)


def test_long_memory_inputs_carry_state_across_chunks():
    """Why the GPU suite has long-memory cases (tests/test_gpu_long_memory.py).

    Cutting every document into independent 64-event pieces drops exactly what the
    state scans carry from one chunk to the next.  With the benchmark gates
    g = -softplus(N(0,1)) that changes the outputs by about 9%: what crosses a chunk
    boundary is almost only the last few events before it, since e^{G_C} is about
    e^-50 per chunk.  With g scaled by 2e-3 (about e^-0.1 per chunk) the state holds
    many chunks of history and the outputs change by about 63%, so only such cases
    test the carried state's decay over many scan steps."""
    T, H, D = 320, 2, 32
    q, k, v, g, beta = rand_inputs(T, H, D, seed=61)
    pieces = tuple(range(0, T + 1, 64))
    for scale, lo, hi in ((1.0, 0.05, 0.15), (2e-3, 0.5, math.inf)):
        whole = O.chunk_delta(q, k, v, g * scale, beta, (0, T))
        cut = O.chunk_delta(q, k, v, g * scale, beta, pieces)
        r = float((cut - whole).norm() / whole.norm())
        assert lo < r < hi, (scale, r)


# ---------------------------------------------------------------- chunked == recurrent
@pytest.mark.parametrize("T,bounds", [(1, None), (63, None), (64, None), (65, None), (129, (0, 37, 129)),
                                      (200, (0, 1, 64, 65, 200)), (130, (0, 0, 130, 130))])
@pytest.mark.parametrize("normalize", [True, False])
def test_chunked_equals_recurrent(T, bounds, normalize):
    q, k, v, g, beta = rand_inputs(T, 2, 16, seed=T)
    n_docs = len(bounds) - 1 if bounds else 1
    s0 = torch.randn(n_docs, 2, 16, 16, dtype=F64, generator=torch.Generator().manual_seed(6)) * 0.1
    ref = O.recurrent_delta(q, k, v, g, beta, bounds, normalize=normalize, initial_state=s0,
                            output_final_state=True)
    got = O.chunk_delta(q, k, v, g, beta, bounds, normalize=normalize, initial_state=s0, output_final_state=True)
    for a, b in zip(got, ref):
        torch.testing.assert_close(a, b, rtol=1e-10, atol=1e-10)


def test_chunk_intermediates_against_independent_forms():
    T, H, D = 100, 2, 16
    q, k, v, g, beta = rand_inputs(T, H, D, seed=7)
    _, _, inter = O.chunk_delta(q, k, v, g, beta, output_final_state=True, return_intermediates=True)
    kn = inter["kn"][0].transpose(0, 1)  # [H,T,D]
    # per-event recurrence, recording the state entering every event and beta*(v - (e^g S)^T k)
    S = torch.zeros(H, D, D, dtype=F64)
    entering, residual = [], []
    for t in range(T):
        entering.append(S.clone())
        S = S * g[0, t].exp()[:, None, None]
        r = v[0, t] - torch.einsum("hkv,hk->hv", S, kn[:, t])
        residual.append(beta[0, t][:, None] * r)
        S = S + beta[0, t][:, None, None] * kn[:, t, :, None] * r[:, None, :]
    for c, (a, b) in enumerate(inter["spans"]):
        n = b - a
        # gcum: running sum within the chunk
        torch.testing.assert_close(inter["gcum"][c], g[0, a:b].transpose(0, 1).cumsum(-1))
        # T = (I + A)^-1 by a different routine than the oracle's triangular solve
        eye = torch.eye(n, dtype=F64)
        torch.testing.assert_close(inter["T"][c], torch.linalg.inv(eye + inter["A"][c]), rtol=1e-9, atol=1e-11)
        assert torch.all(inter["A"][c].triu() == 0)  # strictly lower
        # h: the recurrent state at the chunk start; v_new: beta * residual of each event
        torch.testing.assert_close(inter["h"][c], entering[a], rtol=1e-10, atol=1e-12)
        torch.testing.assert_close(inter["vn"][c], torch.stack(residual[a:b], dim=1), rtol=1e-9, atol=1e-11)


# ---------------------------------------------------------------- invariants
def test_readonly_events_leave_state_and_other_outputs_bit_identical():
    T, H, D = 90, 2, 16
    q, k, v, g, beta = rand_inputs(T, H, D, seed=8)
    ro = torch.zeros(T, dtype=torch.bool)
    ro[30:50] = True
    k2, v2, g2, b2 = k.clone(), v.clone(), g.clone(), beta.clone()
    k2[:, ro], v2[:, ro], g2[:, ro], b2[:, ro] = 0, 0, 0, 0
    o_full, s_full = O.chunk_delta(q, k2, v2, g2, b2, output_final_state=True)
    keep = ~ro
    o_skip, s_skip = O.chunk_delta(q[:, keep], k[:, keep], v[:, keep], g[:, keep], beta[:, keep],
                                   output_final_state=True)
    torch.testing.assert_close(s_full, s_skip, rtol=1e-10, atol=1e-12)
    torch.testing.assert_close(o_full[:, keep], o_skip, rtol=1e-10, atol=1e-12)
    # changing what read-only events query changes only their own outputs
    q3 = q.clone()
    q3[:, ro] = torch.randn_like(q3[:, ro])
    o3, s3 = O.recurrent_delta(q3, k2, v2, g2, b2, output_final_state=True)
    o1, s1 = O.recurrent_delta(q, k2, v2, g2, b2, output_final_state=True)
    assert torch.equal(o3[:, keep], o1[:, keep]) and torch.equal(s3, s1)


def test_documents_are_isolated():
    T, H, D = 150, 2, 16
    bounds = (0, 70, 150)
    q, k, v, g, beta = rand_inputs(T, H, D, seed=9)
    o, s = O.chunk_delta(q, k, v, g, beta, bounds, output_final_state=True)
    o2, s2 = O.chunk_delta(q[:, 70:], k[:, 70:], v[:, 70:], g[:, 70:], beta[:, 70:], output_final_state=True)
    torch.testing.assert_close(o[:, 70:], o2, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(s[1:], s2, rtol=1e-12, atol=1e-12)


def test_chunk_local_cumsum_and_spans():
    g = torch.randn(1, 150, 3, dtype=F64)
    bounds = (0, 10, 150)
    spans = O.chunk_spans(bounds)
    assert spans == [(0, 10), (10, 74), (74, 138), (138, 150)]
    fwd, rev = O.chunk_local_cumsum(g, bounds), O.chunk_local_cumsum(g, bounds, reverse=True)
    for a, b in spans:
        for t in range(a, b):
            torch.testing.assert_close(fwd[:, t], g[:, a:t + 1].sum(1))
            torch.testing.assert_close(rev[:, t], g[:, t:b].sum(1))


def test_decode_step_equals_recurrence_with_transposed_state():
    N, E, H, D = 3, 4, 2, 16
    gen = torch.Generator().manual_seed(10)
    q = O.l2norm(torch.randn(N, E, H, D, dtype=F64, generator=gen))
    k = O.l2norm(torch.randn(N, E, H, D, dtype=F64, generator=gen))
    v = torch.randn(N, E, H, D, dtype=F64, generator=gen)
    g = -torch.nn.functional.softplus(torch.randn(N, E, H, dtype=F64, generator=gen))
    beta = torch.rand(N, E, H, dtype=F64, generator=gen)
    s0 = torch.randn(N, H, D, D, dtype=F64, generator=gen) * 0.02  # value-first
    state = s0.clone()
    out = O.decode_step(q, k, v, g, beta, state)
    for n in range(N):
        o, s = O.recurrent_delta(q[n:n + 1], k[n:n + 1], v[n:n + 1], g[n:n + 1], beta[n:n + 1], normalize=False,
                                 initial_state=s0[n:n + 1].transpose(-1, -2), output_final_state=True)
        torch.testing.assert_close(out[n:n + 1], o, rtol=1e-12, atol=1e-12)
        torch.testing.assert_close(state[n:n + 1], s.transpose(-1, -2), rtol=1e-12, atol=1e-12)


def test_error_stats_semantics():
    # relative L2 with an absolute escape of 2e-7 (scripts/validation/delta64_probe.py:90-99)
    b = torch.ones(4)
    assert O.error_stats(b * 1.01, b, 0.02)["passed"]
    assert not O.error_stats(b * 1.03, b, 0.02)["passed"]
    assert O.error_stats(torch.full((4,), 1e-7), torch.zeros(4), 0.02)["passed"]
    assert not O.error_stats(torch.tensor([float("nan")]), torch.ones(1), 0.02)["passed"]


# ---------------------------------------------------------------- gradients
def test_recurrence_gradcheck():
    q, k, v, g, beta = (x.requires_grad_() for x in rand_inputs(5, 1, 4, seed=11))
    assert torch.autograd.gradcheck(lambda *xs: O.recurrent_delta(*xs, (0, 2, 5)), (q, k, v, g, beta),
                                    eps=1e-6, atol=1e-7)


@pytest.mark.parametrize("T,bounds,normalize", [(1, None, True), (65, None, True), (129, (0, 37, 129), True),
                                                (150, (0, 64, 70, 150), False)])
def test_manual_backward_matches_autograd_of_recurrence(T, bounds, normalize):
    xs = rand_inputs(T, 2, 16, seed=100 + T)
    do = torch.randn(1, T, 2, 16, dtype=F64, generator=torch.Generator().manual_seed(12))
    leaves = [x.clone().requires_grad_() for x in xs]
    O.recurrent_delta(*leaves, bounds, normalize=normalize).backward(do)
    got = O.chunk_delta_backward(*xs, do, bounds, normalize=normalize)
    for name, a, leaf in zip(("dq", "dk", "dv", "dg", "dbeta"), got, leaves):
        torch.testing.assert_close(a, leaf.grad, rtol=1e-9, atol=1e-10, msg=name)


# ---------------------------------------------------------------- planted mistakes
def test_planted_transposed_ut_inverse_is_caught(monkeypatch):
    q, k, v, g, beta = rand_inputs(100, 2, 16, seed=13)
    ref = O.recurrent_delta(q, k, v, g, beta)
    solve = torch.linalg.solve_triangular
    monkeypatch.setattr(torch.linalg, "solve_triangular",
                        lambda *a, **kw: solve(*a, **kw).transpose(-1, -2).contiguous())
    wrong = O.chunk_delta(q, k, v, g, beta)
    assert (wrong - ref).abs().max() > 1e-3


def test_planted_decay_sign_is_caught():
    # flipping the sign of g must break the golden comparison (g enters through exp)
    gv = json.loads((GOLDEN / "recurrence_d8.json").read_text())
    q, k, v = (torch.tensor(gv[n], dtype=F64)[None] for n in ("q", "k", "v"))
    g, beta = (torch.tensor(gv[n], dtype=F64)[None] for n in ("g", "beta"))
    o = O.recurrent_delta(q, k, v, -g, beta, tuple(gv["bounds"]))
    assert (o - torch.tensor(gv["o"], dtype=F64)[None]).abs().max() > 1e-3


def test_planted_backward_mistake_is_caught(monkeypatch):
    # a dropped term in the manual backward (the beta factor of dv) must fail the autograd comparison
    xs = rand_inputs(70, 1, 8, seed=14)
    do = torch.randn(1, 70, 1, 8, dtype=F64, generator=torch.Generator().manual_seed(15))
    leaves = [x.clone().requires_grad_() for x in xs]
    O.recurrent_delta(*leaves).backward(do)
    dq, dk, dv, dg, db = O.chunk_delta_backward(*xs, do)
    torch.testing.assert_close(dv, leaves[2].grad, rtol=1e-9, atol=1e-10)
    wrong_dv = dv / xs[4][..., None]  # the same dv without its beta factor
    assert (wrong_dv - leaves[2].grad).abs().max() > 1e-3


def test_causal_conv1d_closed_form_and_documents():
    """The conv oracle against a scalar loop (row t sees rows t-K+1..t of its own document),
    with and without SiLU, K = 2..4; a planted off-by-one (seeing the next row) is caught."""
    gen = torch.Generator().manual_seed(7)
    for K in (2, 3, 4):
        x = torch.randn(1, 11, 3, generator=gen, dtype=F64)
        w = torch.randn(3, K, generator=gen, dtype=F64)
        bounds = (0, 1, 3, 11)
        want = torch.zeros_like(x)
        for a, b in zip(bounds, bounds[1:]):
            for t in range(a, b):
                for c in range(3):
                    want[0, t, c] = sum(w[c, i] * x[0, t - (K - 1) + i, c] for i in range(K) if t - (K - 1) + i >= a)
        assert torch.allclose(O.causal_conv1d(x, w, bounds, activation=False), want, atol=1e-12)
        assert torch.allclose(O.causal_conv1d(x, w, bounds), torch.nn.functional.silu(want), atol=1e-12)
        shifted = torch.zeros_like(x)
        shifted[:, :-1] = x[:, 1:]
        assert not torch.allclose(O.causal_conv1d(shifted, w, bounds, activation=False), want, atol=1e-6)


def test_gated_rms_norm_against_library_and_closed_form():
    """The gated-norm oracle against torch's own rms_norm times silu (a library routine) and the
    closed form of a constant row (x = c: the norm is c / sqrt(c^2 + eps)); a planted mistake
    (normalizing over the sum instead of the mean) is caught."""
    gen = torch.Generator().manual_seed(11)
    y = torch.randn(5, 3, 128, generator=gen, dtype=F64)
    z = torch.randn(5, 3, 128, generator=gen, dtype=F64)
    w = torch.randn(128, generator=gen, dtype=F64)
    want = torch.nn.functional.rms_norm(y, (128,), w, eps=1e-6) * torch.nn.functional.silu(z)
    assert torch.allclose(O.gated_rms_norm(y, z, w), want, atol=1e-12)
    c = torch.full((1, 128), -0.25, dtype=F64)
    ones = torch.ones(128, dtype=F64)
    closed = -0.25 / (0.0625 + 1e-6) ** 0.5 * torch.nn.functional.silu(z[0, :1])
    assert torch.allclose(O.gated_rms_norm(c, z[0, :1], ones), closed, atol=1e-12)
    planted = y * torch.rsqrt(y.square().sum(-1, keepdim=True) + 1e-6) * w * torch.nn.functional.silu(z)
    assert not torch.allclose(planted, want, atol=1e-3)


@pytest.mark.parametrize("H,HK", [(4, 4), (8, 4)])
def test_layer_decode_step_equals_the_training_layer_on_the_extended_plan(H, HK):
    """Prefill (state after the committed rows, conv history = the K-1 raw rows before the
    uncommitted target, models/backbone_qwen35.py:201-209) followed by one oracle decode step
    equals the training-path layer (the reference's layer code in float64 with the oracle conv,
    recurrence and norm) on the plan where the step's content token commits and its query reads
    after it: the C and Q outputs and the final state, with equal key and value heads and with
    two value heads per key head (the reference's repeat_interleave on both paths).  A planted
    history without the shift (Q's conv not seeing C) is caught."""
    import layer_harness as layer
    from gdn_testlib import decode_plans

    torch.manual_seed(9)
    n, K = 20, 4
    S, SK = H * 128, HK * 128
    C = 2 * SK + S
    model = layer.GatedDeltaLayer(width=32, heads=H, key_heads=HK).double()
    with torch.no_grad():
        model.dt_bias.copy_(torch.randn(H) * 0.5)
        model.norm_weight.copy_(1 + 0.1 * torch.randn(128))
    pre_plan, one_plan = decode_plans(n, K)
    proj = torch.randn(n + 2, C + S + 2 * H, dtype=F64) * 0.7
    cv = lambda u, w, bounds: O.causal_conv1d(u, w, bounds)
    norm = O.gated_rms_norm
    states = {}

    def rec(q, k, v, g, b, p):
        o, st = O.recurrent_delta(q, k, v, g, b, p.event_bounds, normalize=True, output_final_state=True)
        states[len(p.event_q)] = st
        return o

    model.core(proj[:n + 1], pre_plan, recurrence=rec, conv=cv, norm=norm, fused=False)
    want = model.core(proj, one_plan, recurrence=rec, conv=cv, norm=norm, fused=False)
    state0 = states[n + 1].transpose(-1, -2)  # value-first
    history = proj[None, n - K + 1:n, :C]
    rows = proj[None, n:n + 2]
    args = (rows[..., :C], rows[..., C:C + S].reshape(1, 2, H, 128), rows[..., C + S:C + S + H],
            rows[..., C + S + H:], model.conv_weight, model.A_log, model.dt_bias, model.norm_weight)
    out, hist, state = O.layer_decode_step(*args, history, state0)
    assert torch.allclose(out.reshape(2, S), want[n:n + 2], atol=1e-10)
    assert torch.allclose(state[0], states[n + 2][0].transpose(-1, -2), atol=1e-10)
    assert torch.equal(hist[0], proj[n - K + 2:n + 1, :C])
    # planted: Q's conv over the history before C entered it
    hist_old = proj[n - K + 1:n, :SK]
    w = model.conv_weight[:SK]
    wrong_q = torch.nn.functional.silu(proj[n + 1, :SK] * w[:, -1] + sum(hist_old[j] * w[:, j] for j in range(K - 1)))
    right_q = torch.nn.functional.silu(proj[n + 1, :SK] * w[:, -1] +
                                       sum(hist[0, j, :SK] * w[:, j] for j in range(K - 1)))
    assert not torch.allclose(wrong_q, right_q, atol=1e-3)
