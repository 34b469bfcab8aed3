"""Brute-force float64 SRW forward with explicit per-unit Python loops.

TEST INFRASTRUCTURE ONLY.  An independent formulation of the layer (no
matrix products, no torch): every score, moment, gate and output element
is accumulated one term at a time with the ``math`` module, following the
definitions in models/dawn_spatial_v41_exp.py:1713-1738 (v4.1) and
models/legacy/dawn_spatial_v401_exp.py:1443-1463 (v4.0.1).  Used on tiny
inputs (T <= 8, N <= 64, D <= 16) to pin the oracle's vectorised
restatement.
"""

from __future__ import annotations

import math


def _sigmoid(v: float) -> float:
    if v >= 0:
        return 1.0 / (1.0 + math.exp(-v))
    ev = math.exp(v)
    return ev / (1.0 + ev)


def srw_token(x, h, emb, tau_offset, read, write, *, gate="v41", sharpness=500.0,
              act_threshold=0.5, act_cutoff=0.01, epsilon=1e-4, max_intensity=10.0,
              onepass=False):
    """One token.  x [D], h [dr], emb [N][dr], read/write [N][D] (lists of floats).

    Returns dict(out [D], den, gate_sum, int_sum, n_active, tau, s_mean,
    s_std, margins [N], gates [N]).
    """
    N = len(emb)
    D = len(x)
    scores = []
    for n in range(N):
        acc = 0.0
        for k in range(len(h)):
            acc += h[k] * emb[n][k]
        scores.append(acc)
    mean = sum(scores) / N
    if onepass:
        var = sum(s * s for s in scores) / N - mean * mean
    else:
        var = sum((s - mean) ** 2 for s in scores) / N
    std = math.sqrt(var) + 1e-8
    tau = mean + tau_offset * std
    gates, margins, ints = [], [], []
    n_active = 0
    for s in scores:
        if gate == "v41":
            m = (s - tau) - act_threshold
            act = _sigmoid(sharpness * m)
            inten = epsilon + min(max(m - act_cutoff, 0.0), max_intensity)
            g = act * inten
            n_active += act > 0.5
        else:
            m = s - tau
            z = m / std
            phi = 0.5 * (1.0 + math.erf(z / math.sqrt(2.0)))
            g = z * phi if z > 0 else 0.0
            inten = g
            n_active += g > 0.0
        margins.append(m)
        gates.append(g)
        ints.append(inten)
    rn = list(read)
    wn = list(write)
    if gate != "v41":
        rn = [[v / (math.sqrt(sum(u * u for u in row)) + 1e-8) for v in row] for row in read]
        wn = [[v / (math.sqrt(sum(u * u for u in row)) + 1e-8) for v in row] for row in write]
    out = [0.0] * D
    for n in range(N):
        xr = 0.0
        for d in range(D):
            xr += x[d] * rn[n][d]
        c = gates[n] * xr
        for d in range(D):
            out[d] += c * wn[n][d]
    gate_sum = sum(gates)
    int_sum = sum(ints)
    den = max(int_sum if gate == "v41" else gate_sum, 1.0)
    return dict(out=[v / den for v in out], den=den, gate_sum=gate_sum, int_sum=int_sum,
                n_active=n_active, tau=tau, s_mean=mean, s_std=std, margins=margins,
                gates=gates)
