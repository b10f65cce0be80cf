"""Why the A_log and dt_bias gradients are gated by a conditioned error, shown on the CPU.

dA_log[h] = sum_t dg[t,h] * g[t,h] and ddt_bias[h] = sum_t dg[t,h] * (-exp(A_log[h]) * sigmoid(a[t,h] + dt_bias[h]))
are sums of signed per-event terms.  In a head whose terms nearly cancel (condition
kappa_h = sum_t |c_t| / |sum_t c_t| of tens to hundreds), a relative error eps in the per-event dg
becomes an error of about eps * kappa_h in that head's gradient, whatever computes the sum.

The test takes the float64 layer restatement (the reference's layer code with the oracle's conv,
chunked recurrence and norm) on the two-branch plan and head count of
test_layer_core_shared_hidden_rows, draws A_log as the reference module does
(rand * 15.99 + 0.01, then log; models/backbone_qwen35.py:137-141), and compares it with the same
float64 computation in which only the recurrence's inputs and outputs are rounded to bf16 where the
kernels store them (q, k, v and the output y; dy, dq, dk, dv in the backward).  No kernel runs.
Those roundings alone move the raw max-relative error of d_A_log past 2e-2 on some draws, while the
reference's conditioned error (scripts/validation/validate_qwen35_cq.py:84-101: the error norm over
the norm of sum_t |c_t|) stays below 2e-3, and every head's error over its sum of absolute terms
stays below 5e-3.  So a raw relative gate on these two gradients measures the cancellation of the
draw, not the implementation; the GPU tests gate them as the reference does (gdn_testlib.TOL_CONTROL).
"""

import torch

import layer_harness as layer
from oracle import gdn_oracle as O


class _Bf16(torch.autograd.Function):
    """Round to bf16 in the forward and the gradient to bf16 in the backward (float64 in and out)."""

    @staticmethod
    def forward(ctx, x):
        return x.bfloat16().double()

    @staticmethod
    def backward(ctx, dy):
        return dy.bfloat16().double()


def _run(model, plan, proj, dout, rounded):
    captured = {}

    def recurrence(q, k, v, g, b, p):
        g.retain_grad()
        captured["g"] = g
        if rounded:
            r = _Bf16.apply
            return r(O.chunk_delta(r(q), r(k), r(v), g, b, p.event_bounds, normalize=True))
        return O.chunk_delta(q, k, v, g, b, p.event_bounds, normalize=True)

    model.zero_grad(set_to_none=True)
    p64 = proj.double().requires_grad_()
    out = model.core(p64, plan, recurrence=recurrence, conv=lambda u, w, bounds: O.causal_conv1d(u, w, bounds),
                     norm=O.gated_rms_norm, fused=False)
    out.backward(dout.double())
    g = captured["g"]
    return model.A_log.grad.clone(), model.dt_bias.grad.clone(), (g.grad * g.detach())[0]


def test_a_log_raw_error_follows_cancellation_not_the_sum():
    torch.set_num_threads(min(8, torch.get_num_threads()))
    H = 16
    plan = layer.two_branch_plan(260, 70, prefix=40, suffix=50, image_groups=(30,), seed=9)
    worst_raw, report = 0.0, []
    for draw in range(4):
        gen = torch.Generator().manual_seed(91)
        proj = (torch.randn(plan.hidden_length, 4 * H * 128 + 2 * H, generator=gen) * 0.7).bfloat16()
        model = layer.GatedDeltaLayer(width=64, heads=H).double()
        with torch.no_grad():
            model.conv_weight.copy_((torch.rand(model.conv_weight.shape, generator=gen) - 0.5).bfloat16().double())
            model.A_log.copy_(torch.rand(H, generator=torch.Generator().manual_seed(draw)).mul(15.99).add(0.01).log())
            model.dt_bias.copy_(torch.randn(H, generator=gen) * 0.5)
            model.norm_weight.copy_(1 + 0.1 * torch.randn(128, generator=gen))
        dout = (torch.randn(plan.hidden_length, H * 128, generator=gen) * 0.1).bfloat16()
        exact_a, exact_dt, terms = _run(model, plan, proj, dout, rounded=False)
        round_a, round_dt, _ = _run(model, plan, proj, dout, rounded=True)
        absum = terms.abs().sum(0)  # per head, sum_t |dg * g|
        kappa = absum / terms.sum(0).abs()
        raw = float(((round_a - exact_a).abs() / exact_a.abs()).max())
        conditioned = float((round_a - exact_a).norm() / absum.norm())
        per_head = float(((round_a - exact_a).abs() / absum).max())
        worst_raw = max(worst_raw, raw)
        report.append((draw, raw, conditioned, per_head, float(kappa.max())))
        print(f"draw {draw}: d_A_log raw max_rel={raw:.2e} conditioned={conditioned:.2e} "
              f"max_h |err|/sum|terms|={per_head:.2e} max kappa={float(kappa.max()):.0f}", flush=True)
        assert conditioned < 2e-3 and per_head < 5e-3
        # the summed terms reproduce the restatement's own gradient: the cancellation is the sum's
        assert torch.allclose(terms.sum(0), exact_a, rtol=1e-9, atol=1e-12)
    assert worst_raw > 2e-2, report
