"""Write the golden vectors of tests/golden/ with plain-Python arithmetic (no torch, no oracle).

The reference holds no committed golden vectors for the GDN path, so these are
written from the per-event gated delta rule itself (models/backbone_qwen35.py:56-72:
l2norm q and k, q *= d^-1/2; per event S <- exp(g) S; r = v - S^T k;
S <- S + beta k r^T; o = S^T q; state reset at each document start), evaluated
with Python floats in a scalar loop, and of the value-first decode step
(models/decoding.py:71-77).  The CPU tests compare the torch oracle with them.

Run from the repository root:  python tests/golden/make_golden.py
"""

import json
import math
import random
from pathlib import Path

HERE = Path(__file__).resolve().parent


def l2norm(x, eps=1e-6):
    r = 1.0 / math.sqrt(sum(a * a for a in x) + eps)
    return [a * r for a in x]


def recurrence(q, k, v, g, beta, bounds, d):
    """q,k,v: [T][H][d]; g, beta: [T][H].  Returns o [T][H][d] and final states [N][H][d][d] (key-first)."""
    T, H = len(q), len(q[0])
    scale = d ** -0.5
    o = [[None] * H for _ in range(T)]
    finals = []
    for a, b in zip(bounds, bounds[1:]):
        S = [[[0.0] * d for _ in range(d)] for _ in range(H)]
        for t in range(a, b):
            for h in range(H):
                qn = [x * scale for x in l2norm(q[t][h])]
                kn = l2norm(k[t][h])
                decay = math.exp(g[t][h])
                Sh = S[h]
                for i in range(d):
                    for j in range(d):
                        Sh[i][j] *= decay
                r = [v[t][h][j] - sum(Sh[i][j] * kn[i] for i in range(d)) for j in range(d)]
                for i in range(d):
                    for j in range(d):
                        Sh[i][j] += beta[t][h] * kn[i] * r[j]
                o[t][h] = [sum(Sh[i][j] * qn[i] for i in range(d)) for j in range(d)]
        finals.append([[row[:] for row in S[h]] for h in range(H)])
    return o, finals


def decode(q, k, v, g, beta, state, d):
    """Value-first state [N][H][V][K], events [N][E][H][d]; q,k already normalized.  In place."""
    scale = d ** -0.5
    N, E, H = len(q), len(q[0]), len(q[0][0])
    out = [[[None] * H for _ in range(E)] for _ in range(N)]
    for n in range(N):
        for e in range(E):
            for h in range(H):
                S = state[n][h]
                decay = math.exp(g[n][e][h])
                for i in range(d):
                    for j in range(d):
                        S[i][j] *= decay
                r = [v[n][e][h][i] - sum(S[i][j] * k[n][e][h][j] for j in range(d)) for i in range(d)]
                for i in range(d):
                    for j in range(d):
                        S[i][j] += beta[n][e][h] * r[i] * k[n][e][h][j]
                out[n][e][h] = [scale * sum(S[i][j] * q[n][e][h][j] for j in range(d)) for i in range(d)]
    return out


def rnd(rng, *shape, f=lambda r: round(r.gauss(0, 1), 4)):
    if not shape:
        return f(rng)
    return [rnd(rng, *shape[1:], f=f) for _ in range(shape[0])]


def sigmoid(x):
    return 1.0 / (1.0 + math.exp(-x))


def softplus(x):
    return math.log1p(math.exp(x))


def main():
    rng = random.Random(20261201)
    d, H, T = 8, 2, 70
    bounds = [0, 5, 70]  # a short document, then one crossing the 64-event chunk boundary
    q, k, v = rnd(rng, T, H, d), rnd(rng, T, H, d), rnd(rng, T, H, d)
    g = rnd(rng, T, H, f=lambda r: round(-softplus(r.gauss(0, 1)), 4))
    beta = rnd(rng, T, H, f=lambda r: round(sigmoid(r.gauss(0, 1)), 4))
    readonly = list(range(20, 28))  # read-only query events: real q, k = v = 0, g = beta = 0
    for t in readonly:
        for h in range(H):
            k[t][h] = [0.0] * d
            v[t][h] = [0.0] * d
            g[t][h] = 0.0
            beta[t][h] = 0.0
    o, finals = recurrence(q, k, v, g, beta, bounds, d)
    (HERE / "recurrence_d8.json").write_text(json.dumps(dict(
        description="per-event gated delta rule, plain-Python floats; q,k l2-normalized inside, scale d^-1/2",
        d=d, H=H, T=T, bounds=bounds, readonly=readonly, q=q, k=k, v=v, g=g, beta=beta, o=o, final_state=finals)))

    N, E = 2, 2
    qd = [[[l2norm(x) for x in ev] for ev in seq] for seq in rnd(rng, N, E, H, d)]
    kd = [[[l2norm(x) for x in ev] for ev in seq] for seq in rnd(rng, N, E, H, d)]
    vd = rnd(rng, N, E, H, d)
    gd = rnd(rng, N, E, H, f=lambda r: round(-softplus(r.gauss(0, 1)), 4))
    bd = rnd(rng, N, E, H, f=lambda r: round(sigmoid(r.gauss(0, 1)), 4))
    state0 = rnd(rng, N, H, d, d, f=lambda r: round(0.02 * r.gauss(0, 1), 5))
    state = json.loads(json.dumps(state0))
    out = decode(qd, kd, vd, gd, bd, state, d)
    (HERE / "decode_d8.json").write_text(json.dumps(dict(
        description="value-first decode step, plain-Python floats; q,k given normalized; state updated in place",
        d=d, H=H, N=N, E=E, q=qd, k=kd, v=vd, g=gd, beta=bd, state_in=state0, state_out=state, out=out)))


if __name__ == "__main__":
    main()
