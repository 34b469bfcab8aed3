"""Pin the CPU oracle (oracle/srw_ref.py) before trusting it.

The reference ships no tests or golden vectors for the SRW path, so every
check here is against something the mathematics fixes: closed forms, a
brute-force float64 per-unit loop (oracle/brute.py), textbook / library
routines (scipy), exact rounding cases and invariants.  The last group
plants mistakes in the oracle and asserts that these pins catch them.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import scipy.optimize
import scipy.special
import scipy.stats
import torch

from oracle import brute, srw_ref

F64 = torch.float64
F32 = torch.float32
BF = torch.bfloat16


def _rand_inputs(T, D, dr, N, seed, dtype=F64, tau=-0.5):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, D, generator=g, dtype=F64)
    x = x / torch.sqrt((x * x).mean(-1, keepdim=True) + 1e-6)
    h = torch.randn(T, dr, generator=g, dtype=F64)
    e = torch.randn(N, dr, generator=g, dtype=F64) / math.sqrt(dr)
    r = torch.randn(N, D, generator=g, dtype=F64)
    r = r / r.norm(dim=-1, keepdim=True)
    w = torch.randn(N, D, generator=g, dtype=F64)
    w = w / w.norm(dim=-1, keepdim=True)
    tau_off = torch.full((T, 1), tau, dtype=F64)
    return [t.to(dtype) for t in (x, h, e, tau_off, r, w)]


# ---------------------------------------------------------------- gates

def test_gate_v41_closed_form_grid():
    m64 = torch.cat([torch.linspace(-1.0, 12.0, 20001, dtype=F64),
                     torch.tensor([0.0, 0.01, 10.01, 1e-3, -1e-3], dtype=F64)])
    tau = torch.zeros((), dtype=F32)
    s = (m64 + 0.5).to(F32)                 # score such that margin = s - 0 - 0.5
    margin, act, inten, gate = srw_ref.gate_v41(s, tau)
    m = margin.to(F64)
    act64 = 1.0 / (1.0 + torch.exp(-500.0 * m))
    int64 = 1e-4 + torch.clamp(m - 0.01, 0.0, 10.0)
    # fp32 rounding of the sigmoid argument 500 m costs |500 m| * 2^-23 relative
    bound = act64 * (1e-6 + (500.0 * m).abs() * 2.0 ** -23) + 1e-37
    assert torch.all((act.to(F64) - act64).abs() <= bound)
    assert torch.allclose(inten.to(F64), int64, rtol=1e-6, atol=1e-7)
    assert torch.all((gate.to(F64) - act64 * int64).abs() <= bound * int64 * 1.01 + 1e-37)
    eps32 = torch.tensor(1e-4, dtype=F32)
    assert torch.all(inten[margin <= torch.tensor(0.01, dtype=F32)] == eps32)   # intensity == eps exactly
    cap = (eps32 + torch.tensor(10.0, dtype=F32))
    assert torch.all(inten[m >= 10.02] == cap)                                 # cap
    away = m.abs() > 1e-6
    assert torch.equal((act > 0.5)[away], (m > 0)[away])                        # act > .5 <=> margin > 0


def test_gate_gelu_v401_closed_form_grid():
    z64 = torch.linspace(-6.0, 6.0, 12001, dtype=F64)
    std = torch.tensor(1.7, dtype=F32)
    raw = (z64 * 1.7).to(F32)
    z, phi, gate = srw_ref.gate_gelu_v401(raw, std)
    zz = z.to(F64).numpy()
    expect = np.where(zz > 0, zz * scipy.special.ndtr(zz), 0.0)
    assert np.allclose(gate.to(F64).numpy(), expect, rtol=2e-6, atol=1e-12)
    assert torch.all(gate[z <= 0] == 0)


# ---------------------------------------------------------------- brute force

@pytest.mark.parametrize("seed", [0, 1, 2])
@pytest.mark.parametrize("gate", ["v41", "gelu_v401"])
def test_oracle_fp64_matches_brute_force(seed, gate):
    T, D, dr, N = 5, 12, 8, 40
    x, h, e, tau, r, w = _rand_inputs(T, D, dr, N, seed, tau=-0.5 if gate == "v41" else 0.4)
    if gate == "v41":
        out, tr = srw_ref.srw_inference(x, h, e, tau, r, w, acc_dtype=F64, return_trace=True)
    else:
        out, tr = srw_ref.srw_inference_gelu_v401(x, h, e, tau, r, w, acc_dtype=F64,
                                                  return_trace=True)
    for t in range(T):
        b = brute.srw_token(x[t].tolist(), h[t].tolist(), e.tolist(), float(tau[t, 0]),
                            r.tolist(), w.tolist(), gate=gate)
        assert np.allclose(out[t].numpy(), b["out"], rtol=1e-10, atol=1e-13)
        assert math.isclose(float(tr["den"][t, 0]), b["den"], rel_tol=1e-12)
        assert math.isclose(float(tr["tau"][t, 0]), b["tau"], rel_tol=1e-12, abs_tol=1e-14)
        assert np.allclose(tr["gate"][t].numpy(), b["gates"], rtol=1e-10, atol=1e-15)


def test_onepass_stats_match_brute_force():
    """fused_gate_srw's one-pass s_std (v41:461-462) vs a float64 loop on the same bf16 scores."""
    T, D, dr, N = 4, 16, 16, 64
    x, h, e, tau, r, w = _rand_inputs(T, D, dr, N, 7, dtype=F32)
    st = srw_ref._pass1_stats(h.to(BF)[None], e.to(BF), 1, N, N, route_axis=False)
    scores = srw_ref.dot_bf16(h.to(BF), e.to(BF)).to(F64)
    for t in range(T):
        s = scores[t].tolist()
        mean = sum(s) / N
        std = math.sqrt(sum(v * v for v in s) / N - mean * mean) + 1e-8
        assert math.isclose(float(st["s_std"][0, t, 0]), std, rel_tol=2e-6)
        assert math.isclose(float(st["s_mean"][0, t, 0]), mean, rel_tol=1e-5, abs_tol=1e-7)


def test_gram_identity():
    """sum_n s = h . (sum_n e_n), sum_n s^2 = h^T (E^T E) h  (closed form of the moments)."""
    x, h, e, tau, r, w = _rand_inputs(6, 8, 24, 300, 3)
    s = h @ e.T
    assert torch.allclose(s.sum(-1), h @ e.sum(0), rtol=1e-12, atol=1e-12)
    G = e.T @ e
    assert torch.allclose((s * s).sum(-1), ((h @ G) * h).sum(-1), rtol=1e-12)


# ---------------------------------------------------------------- bf16 emulation

def _rne_bf16_np(v: np.ndarray) -> np.ndarray:
    """Round float64 values (exactly representable in float32) to bf16 by bit arithmetic."""
    u = v.astype(np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return (u.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def test_dot_bf16_rounds_to_nearest_even():
    # integer-valued operands: every fp32 partial sum is exact, so the only rounding is the bf16 one
    a = torch.tensor([[257.0, 0.0], [259.0, 0.0], [385.0, 0.0], [1.0, 1.0 / 256]], dtype=BF)
    assert a[0, 0].item() == 256.0  # 257 itself is not bf16; build sums instead
    a = torch.tensor([[256.0, 1.0], [256.0, 3.0], [384.0, 1.0], [1.0, 0.00390625]], dtype=BF)
    b = torch.tensor([[1.0, 1.0]], dtype=BF)
    got = srw_ref.dot_bf16(a, b).to(F64).flatten().numpy()
    exact = (a.to(F64) @ b.to(F64).T).flatten().numpy()           # 257, 259, 385, 1.00390625
    assert list(got) == [256.0, 260.0, 384.0, 1.0]                   # ties to even
    assert np.array_equal(got, _rne_bf16_np(exact))
    g = torch.Generator().manual_seed(0)
    a = torch.randint(-8, 8, (64, 16), generator=g).to(BF)
    b = torch.randint(-8, 8, (32, 16), generator=g).to(BF)
    exact = (a.to(F64) @ b.to(F64).T).numpy()
    assert np.array_equal(srw_ref.dot_bf16(a, b).to(F64).numpy(), _rne_bf16_np(exact))


def test_fused_bf16_close_to_fp64_layer():
    T, D, dr, N = 32, 64, 32, 900
    x, h, e, tau, r, w = _rand_inputs(T, D, dr, N, 4, dtype=F32)
    out64 = srw_ref.srw_inference(*(t.to(F64) for t in (x, h, e, tau, r, w)), acc_dtype=F64)
    res = srw_ref.fused_gate_srw(x[None], h[None], e, tau[None], r, w, max_chunk_size=4096)
    rel = float((res[0][0].to(F64) - out64).norm() / out64.norm())
    assert rel < 1.5e-2
    res_c = srw_ref.fused_gate_srw(x[None], h[None], e, tau[None], r, w, max_chunk_size=300)
    assert srw_ref.chunk_plan(N, 300) == (3, 300)
    relc = float((res_c[0][0] - res[0][0]).norm() / res[0][0].norm())
    assert 0 < relc < 1e-2           # chunking only changes the bf16 rounding of partial outs


@pytest.mark.parametrize("n,mc,expect", [
    (25200, 12500, (2, 12600)), (1580, 12500, (1, 1580)), (2600, 2048, (1, 2600)),
    (7, 2, (7, 1)), (12, 5, (2, 6)), (100000, 12500, (8, 12500)), (25200, 2048, (12, 2100)),
])
def test_chunk_plan(n, mc, expect):
    assert srw_ref.chunk_plan(n, mc) == expect


# ---------------------------------------------------------------- diagnostics

def test_fused_diagnostics_closed_forms():
    T, D, dr, N = 24, 32, 32, 500
    x, h, e, tau, r, w = _rand_inputs(T, D, dr, N, 9, dtype=F32)
    res, tr = srw_ref.fused_gate_srw(x[None], h[None], e, tau[None], r, w,
                                     max_chunk_size=200, return_trace=True)
    names = srw_ref.FUSED_OUTPUT_NAMES
    o = dict(zip(names, res))
    m = tr["margin"][0].to(F64)                       # [T, N]
    far = lambda thr: (m.abs() - thr).abs() > 1e-6    # noqa: E731
    assert far(0.0).all()
    assert torch.equal(tr["n_active"][0, :, 0], (m > 0).sum(-1).to(F32))
    ln = lambda p: math.log(p / (1 - p)) / 500.0      # noqa: E731  act > p <=> m > logit(p)/500
    assert torch.allclose(o["strong_frac"][0, :, 0] * N, (m > ln(0.9)).sum(-1).to(F32))
    assert torch.allclose(o["boundary_frac"][0, :, 0] * N, (m.abs() < ln(0.9)).sum(-1).to(F32))
    n075 = (m.abs() < ln(0.95)).sum(-1).to(F64)
    assert math.isclose(float(o["z_lt_075_frac"]),
                        float((n075 / (m > 0).sum(-1).clamp_min(1)).mean()), rel_tol=1e-5)
    isum = N * 1e-4 + torch.clamp(m - 0.01, 0.0, 10.0).sum(-1)      # closed form of sum intensity
    assert torch.allclose(tr["intensity_sum"][0, :, 0].to(F64), isum, rtol=1e-5)
    # skew / kurtosis of the bf16 scores vs scipy (population moments)
    scores = srw_ref.dot_bf16(h.to(BF), e.to(BF)).to(F64).numpy()
    sk = scipy.stats.skew(scores, axis=-1).mean()
    ku = scipy.stats.kurtosis(scores, axis=-1, fisher=False).mean()
    assert math.isclose(float(o["score_skew"]), sk, rel_tol=1e-3, abs_tol=1e-4)
    assert math.isclose(float(o["score_kurt"]), ku, rel_tol=1e-4)
    # entropy: -sum g log g / G + log G == entropy of g / G
    g = tr["gate"][0].to(F64).numpy()
    ent = scipy.stats.entropy(g, axis=-1).mean()
    assert math.isclose(float(o["gate_entropy"]), ent, rel_tol=1e-4)
    # score LB: variance / (mean^2 + var + 1e-2) of the per-unit mean scores
    pn = scores.mean(axis=0)
    lb = pn.var() / (pn.mean() ** 2 + pn.var() + 1e-2)
    assert math.isclose(float(o["score_lb"]), lb, rel_tol=1e-4, abs_tol=1e-7)
    # active_per_token_std is the population std
    assert math.isclose(float(o["active_per_token_std"]),
                        float((m > 0).sum(-1).to(F64).std(correction=0)), rel_tol=1e-5)


def test_dead_units_planted():
    T, D, dr, N = 16, 32, 32, 300
    x, h, e, tau, r, w = _rand_inputs(T, D, dr, N, 10, dtype=F32, tau=0.5)
    dead = torch.arange(0, N, 37)
    # |score| <= 0.05 |h_t| ~ 0.3 while tau + 0.5 ~ 1: never passes; mean score < 0
    e[dead] = -0.05 * h.mean(0) / h.mean(0).norm()
    res, tr = srw_ref.fused_gate_srw(x[None], h[None], e, tau[None], r, w,
                                     max_chunk_size=100, return_trace=True)
    o = dict(zip(srw_ref.FUSED_OUTPUT_NAMES, res))
    gmax_unit = tr["gate"][0].amax(0)
    assert torch.all(gmax_unit[dead] < 0.01)
    assert float(o["dead_count"]) == float((gmax_unit < 0.01).sum())
    assert float(o["dead_count"]) >= len(dead)
    mean_score = srw_ref.dot_bf16(h.to(BF), e.to(BF)).float().mean(0)
    pen = (torch.relu(-mean_score) * (gmax_unit < 0.01).float()).sum()
    assert math.isclose(float(o["dead_penalty"]), float(pen), rel_tol=1e-5)


def test_intensity_cap_planted():
    T, D, dr, N = 8, 16, 16, 100
    x, h, e, tau, r, w = _rand_inputs(T, D, dr, N, 11, dtype=F32)
    e[:5] = 40.0 * h.mean(0) / h.mean(0).norm() ** 2      # huge positive scores
    res, tr = srw_ref.fused_gate_srw(x[None], h[None], e, tau[None], r, w,
                                     max_chunk_size=4096, return_trace=True)
    o = dict(zip(srw_ref.FUSED_OUTPUT_NAMES, res))
    m = tr["margin"][0]
    capped = (torch.clamp(m - 0.01, 0, 10) + 1e-4 >= 1e-4 + 10.0 - 1e-3).sum()
    assert int(capped) >= 1
    assert math.isclose(float(o["int_cap_frac"]), float(capped) / (T * N), rel_tol=1e-6)
    assert float(o["int_max"]) == float(torch.tensor(1e-4, dtype=F32) + torch.tensor(10.0, dtype=F32))


# ---------------------------------------------------------------- invariants

def test_token_rows_independent():
    T, D, dr, N = 16, 32, 16, 400
    x, h, e, tau, r, w = _rand_inputs(T, D, dr, N, 12)
    full = srw_ref.srw_inference(x, h, e, tau, r, w, acc_dtype=F64)
    parts = torch.cat([srw_ref.srw_inference(x[i:i + 4], h[i:i + 4], e, tau[i:i + 4], r, w,
                                             acc_dtype=F64) for i in range(0, T, 4)])
    assert torch.allclose(full, parts, rtol=1e-12, atol=1e-15)


def test_unit_permutation_equivariance():
    T, D, dr, N = 6, 24, 16, 200
    x, h, e, tau, r, w = _rand_inputs(T, D, dr, N, 13)
    perm = torch.randperm(N, generator=torch.Generator().manual_seed(1))
    a, ta = srw_ref.srw_inference(x, h, e, tau, r, w, acc_dtype=F64, return_trace=True)
    b, tb = srw_ref.srw_inference(x, h, e[perm], tau, r[perm], w[perm], acc_dtype=F64,
                                  return_trace=True)
    assert torch.allclose(a, b, rtol=1e-10, atol=1e-14)
    assert torch.equal(ta["margin"][:, perm] > 0, tb["margin"] > 0)


def test_write_and_read_rows_enter_linearly():
    """Scaling w_k (or r_k) by alpha changes out by exactly (alpha-1) g_k (x.r_k) w_k / den."""
    T, D, dr, N = 5, 20, 12, 90
    x, h, e, tau, r, w = _rand_inputs(T, D, dr, N, 14)
    base, tr = srw_ref.srw_inference(x, h, e, tau, r, w, acc_dtype=F64, return_trace=True)
    k, alpha = 17, 2.5
    contrib = (tr["gate"][:, k] * (x @ r[k]))[:, None] * w[k][None] / tr["den"]
    w2 = w.clone()
    w2[k] *= alpha
    assert torch.allclose(srw_ref.srw_inference(x, h, e, tau, r, w2, acc_dtype=F64) - base,
                          (alpha - 1) * contrib, rtol=1e-9, atol=1e-14)
    r2 = r.clone()
    r2[k] *= alpha
    assert torch.allclose(srw_ref.srw_inference(x, h, e, tau, r2, w, acc_dtype=F64) - base,
                          (alpha - 1) * contrib, rtol=1e-9, atol=1e-14)


def test_paired_equals_two_singles():
    B, S, D, dr, N = 1, 12, 32, 16, 300
    x, h, e, tau, r, w = _rand_inputs(B * S, D, dr, N, 15, dtype=F32)
    h2 = torch.stack([h, torch.flip(h, dims=[1])], dim=1)           # [T, 2, dr]
    tau2 = torch.stack([tau, tau + 0.3], dim=1)                    # [T, 2, 1]
    pr = srw_ref.fused_gate_srw_paired(x[None], h2[None], e, tau2[None], r, w, max_chunk_size=100)
    for k in range(2):
        sg = srw_ref.fused_gate_srw(x[None], h2[:, k][None], e, tau2[:, k][None], r, w,
                                    max_chunk_size=100)
        assert torch.allclose(pr[0][0, :, k], sg[0][0], rtol=0, atol=1e-6)


# Per-token [B,S,1] outputs of the paired 22-tuple: route means (v41:864-871).
_PAIRED_ROUTE_MEAN = ("active_frac", "gate_max", "strong_frac", "boundary_frac", "z_mean_active")


def _paired_vs_single_mismatch(seed=17):
    """The paired call's 22-tuple against ONE single-route call over the
    2*B*S virtual rows (token t, route r) -> row (s, r) of a [B, 2S] batch,
    with x repeated per route.  fused_gate_srw_paired's statistics are all
    per (token, route) row over N (v41:713-763), so that single call holds
    every row of it; its reductions then fix the paired ones:

    * out: the single's rows, route by route (v41:854-860);
    * active / gate-max / strong / boundary fractions and z_mean_active: the
      mean over the two routes of the single's per-row values (v41:864-871);
    * every scalar -- score_lb and the dead-unit penalty / count from per-unit
      means and maxima over (B, S, 2) (v41:725, 817-818), the moments,
      entropy, int_max, and int_cap_frac over B*S*2*N cells (v41:900-901) --
      the single's scalar over its 2*B*S rows.

    The single-route function is pinned against the brute-force loop, closed
    forms and scipy above.  Inputs plant dead units and units capped at
    max_intensity so that dead_count, dead_penalty and int_cap_frac are not
    zero.  Returns the names that disagree."""
    B, S, D, dr, N = 2, 6, 32, 16, 600
    x, h, e, tau, r, w = _rand_inputs(B * S, D, dr, N, seed, dtype=F32, tau=0.0)
    g = torch.Generator().manual_seed(seed + 1)
    h2 = torch.stack([h, torch.randn(B * S, dr, generator=g)], dim=1)      # [T, 2, dr]
    tau2 = torch.stack([tau, tau + 0.4], dim=1)                           # [T, 2, 1]
    hm = h2.mean(dim=(0, 1))
    e[:4] = 25.0 * hm / hm.norm() ** 2                                     # capped intensity
    e[10:600:83] = -0.02 * hm / hm.norm()                                  # dead units
    pr = srw_ref.fused_gate_srw_paired(x.reshape(B, S, D), h2.reshape(B, S, 2, dr), e,
                                       tau2.reshape(B, S, 2, 1), r, w, max_chunk_size=100)
    xs = x.reshape(B, S, 1, D).expand(B, S, 2, D).reshape(B, 2 * S, D)
    sg = srw_ref.fused_gate_srw(xs, h2.reshape(B, 2 * S, dr), e, tau2.reshape(B, 2 * S, 1), r, w,
                                max_chunk_size=100)
    P = dict(zip(srw_ref.FUSED_OUTPUT_NAMES, pr))
    Q = dict(zip(srw_ref.FUSED_OUTPUT_NAMES, sg))
    assert float(Q["dead_count"]) >= 7 and float(Q["int_cap_frac"]) > 0 and float(Q["dead_penalty"]) > 0
    bad = []
    for name in srw_ref.FUSED_OUTPUT_NAMES:
        p, q = P[name], Q[name]
        if name == "out":
            q = q.reshape(B, S, 2, D)
        elif name in _PAIRED_ROUTE_MEAN:
            q = q.reshape(B, S, 2, 1).mean(dim=2)
        if p.shape != q.shape or not torch.allclose(p, q, rtol=2e-5, atol=1e-7):
            bad.append(name)
    return bad


def test_paired_diagnostics_equal_one_single_over_route_rows():
    assert _paired_vs_single_mismatch() == []


PAIRED_MUTATIONS = {
    # per-unit score means taken per route (over (B, S) only) for score_lb
    "score_lb_per_route": ("_unit_means", lambda s, axes: s.mean(dim=axes[:2]), "score_lb"),
    # the cap fraction over B*S*N cells (the single call's count)
    "int_cap_over_BSN": ("_cell_count", lambda B, S, R, N: float(B * S * N), "int_cap_frac"),
    # per-token fractions of route 0 instead of the route mean
    "active_frac_unaveraged": ("_route_mean", lambda t: t[:, :, 0], "active_frac"),
}


@pytest.mark.parametrize("name", sorted(PAIRED_MUTATIONS))
def test_planted_paired_diagnostic_mistakes_are_caught(monkeypatch, name):
    attr, fn, field = PAIRED_MUTATIONS[name]
    monkeypatch.setattr(srw_ref, attr, fn)
    assert field in _paired_vs_single_mismatch()


def test_den_floor_active_for_small_pools():
    T, D, dr, N = 8, 16, 16, 158
    x, h, e, tau, r, w = _rand_inputs(T, D, dr, N, 16, tau=2.5)
    out, tr = srw_ref.srw_inference(x, h, e, tau, r, w, acc_dtype=F64, return_trace=True)
    isum = tr["intensity"].sum(-1)
    assert (isum < 1).any() and torch.all(tr["den"][:, 0] == torch.clamp_min(isum, 1.0))


# ---------------------------------------------------------------- planted mistakes

def _brute_mismatch(monkeypatch_fn=None):
    """True iff the (possibly mutated) oracle disagrees with the brute-force loop."""
    T, D, dr, N = 3, 12, 12, 30
    x, h, e, tau, r, w = _rand_inputs(T, D, dr, N, 99)
    out, tr = srw_ref.srw_inference(x, h, e, tau, r, w, acc_dtype=F64, return_trace=True)
    for t in range(T):
        b = brute.srw_token(x[t].tolist(), h[t].tolist(), e.tolist(), float(tau[t, 0]),
                            r.tolist(), w.tolist())
        if not np.allclose(out[t].numpy(), b["out"], rtol=1e-10, atol=1e-13):
            return True
    return False


MUTATIONS = {
    "threshold_sign": lambda s, tau, c=srw_ref.V41: srw_ref_gate(s, tau, c, thr_sign=-1),
    "no_epsilon": lambda s, tau, c=srw_ref.V41: srw_ref_gate(s, tau, c, eps=0.0),
    "cutoff_dropped": lambda s, tau, c=srw_ref.V41: srw_ref_gate(s, tau, c, cut=0.0),
    "sharpness_off": lambda s, tau, c=srw_ref.V41: srw_ref_gate(s, tau, c, sharp=50.0),
}
_ORIG_GATE = srw_ref.gate_v41


def srw_ref_gate(s, tau, c, thr_sign=1, eps=None, cut=None, sharp=None):
    dt = s.dtype
    margin = (s - tau) - thr_sign * c.activation_threshold
    act = torch.sigmoid((c.sharpness if sharp is None else sharp) * margin)
    am = torch.clamp_min(margin - (c.activation_cutoff if cut is None else cut), 0.0)
    inten = torch.tensor(c.epsilon if eps is None else eps, dtype=dt) + torch.clamp_max(am, c.max_intensity)
    return margin, act, inten, act * inten


def test_pins_accept_unmutated_oracle():
    assert not _brute_mismatch()


@pytest.mark.parametrize("name", sorted(MUTATIONS))
def test_planted_gate_mistakes_are_caught(monkeypatch, name):
    monkeypatch.setattr(srw_ref, "gate_v41", MUTATIONS[name])
    assert _brute_mismatch()


def test_planted_std_epsilon_inside_sqrt_is_caught(monkeypatch):
    orig = srw_ref._srw_inference_core

    def core(x, h, emb, tau_offset, w_read, w_write, c, acc):
        out, tr = orig(x, h, emb, tau_offset, w_read, w_write, c, acc)
        return out, tr
    # mutate: +1e-8 moved inside the sqrt
    def mutated(x, h, emb, tau_offset, w_read, w_write, c, acc):
        scores = h @ emb.T
        sm = scores.mean(-1, keepdim=True)
        sd = torch.sqrt(((scores - sm) ** 2).mean(-1, keepdim=True) + 1e-8)
        tau = sm + tau_offset * sd
        margin, act, inten, gate = _ORIG_GATE(scores, tau, c)
        den = torch.clamp_min(inten.sum(-1, keepdim=True), 1.0)
        return (gate * (x @ w_read.T)) @ w_write / den, dict(den=den, tau=tau, gate=gate)
    monkeypatch.setattr(srw_ref, "_srw_inference_core", mutated)
    assert _brute_mismatch()


def test_planted_den_from_gate_sum_is_caught(monkeypatch):
    def mutated(x, h, emb, tau_offset, w_read, w_write, c, acc):
        scores = h @ emb.T
        sm = scores.mean(-1, keepdim=True)
        sd = torch.sqrt(((scores - sm) ** 2).mean(-1, keepdim=True)) + 1e-8
        tau = sm + tau_offset * sd
        margin, act, inten, gate = _ORIG_GATE(scores, tau, c)
        den = torch.clamp_min(gate.sum(-1, keepdim=True), 1.0)     # wrong: v4.0.1 den
        return (gate * (x @ w_read.T)) @ w_write / den, dict(den=den, tau=tau, gate=gate)
    monkeypatch.setattr(srw_ref, "_srw_inference_core", mutated)
    assert _brute_mismatch()


def test_planted_transposed_operand_is_caught(monkeypatch):
    def mutated(x, h, emb, tau_offset, w_read, w_write, c, acc):
        scores = h @ emb.T
        sm = scores.mean(-1, keepdim=True)
        sd = torch.sqrt(((scores - sm) ** 2).mean(-1, keepdim=True)) + 1e-8
        tau = sm + tau_offset * sd
        margin, act, inten, gate = _ORIG_GATE(scores, tau, c)
        den = torch.clamp_min(inten.sum(-1, keepdim=True), 1.0)
        xr = h @ w_read.T                                          # wrong operand (h for x)
        return (gate * xr) @ w_write / den, dict(den=den, tau=tau, gate=gate)
    monkeypatch.setattr(srw_ref, "_srw_inference_core", mutated)
    assert _brute_mismatch()


# ---------------------------------------------------------------- v4.0.1 fused function
#
# fused_gate_srw_gelu_v401 (v401:230-367) is pinned through its exact-arithmetic
# form (float64, no bf16 rounding): every output against the brute-force loop
# and numpy / scipy closed forms computed from a textbook float64 score matrix;
# its bf16 form against the exact form within the bf16 error budget; planted
# mistakes (den from sum z+, R / W rows not normalised, gate below zero,
# Phi without the 1/sqrt(2)) must fail the brute-force comparison.

def _v401_inputs(seed, T=5, D=12, dr=8, N=40, tau=0.4):
    """Inputs whose R and W rows are NOT unit-norm (scaled by 0.5 .. 2.5), so
    that the forward normalisation of v401:300-301 changes the result."""
    x, h, e, tau_off, r, w = _rand_inputs(T, D, dr, N, seed, tau=tau)
    g = torch.Generator().manual_seed(seed + 1000)
    r = r * (0.5 + 2.0 * torch.rand(N, 1, generator=g, dtype=F64))
    w = w * (0.5 + 2.0 * torch.rand(N, 1, generator=g, dtype=F64))
    return x, h, e, tau_off, r, w


def _v401_exact(x, h, e, tau, r, w, max_chunk):
    return srw_ref.fused_gate_srw_gelu_v401(x[None], h[None], e, tau[None], r, w,
                                            max_chunk_size=max_chunk, exact=True,
                                            return_trace=True)


def _v401_brute_mismatch(seed=5, max_chunk=20):
    """True iff the exact fused v4.0.1 oracle disagrees with the brute-force
    loop (one-pass std, as the fused function's pass 1, v401:272-273)."""
    x, h, e, tau, r, w = _v401_inputs(seed)
    res, tr = _v401_exact(x, h, e, tau, r, w, max_chunk)
    for t in range(x.shape[0]):
        b = brute.srw_token(x[t].tolist(), h[t].tolist(), e.tolist(), float(tau[t, 0]),
                            r.tolist(), w.tolist(), gate="gelu_v401", onepass=True)
        if not (np.allclose(res[0][0, t].numpy(), b["out"], rtol=1e-10, atol=1e-13)
                and math.isclose(float(tr["den"][0, t, 0]), b["den"], rel_tol=1e-12)
                and math.isclose(float(tr["gate_sum"][0, t, 0]), b["gate_sum"], rel_tol=1e-12)):
            return True
    return False


@pytest.mark.parametrize("seed", [5, 6, 7])
@pytest.mark.parametrize("max_chunk", [20, 4096])
def test_fused_v401_exact_matches_brute_force(seed, max_chunk):
    x, h, e, tau, r, w = _v401_inputs(seed)
    res, tr = _v401_exact(x, h, e, tau, r, w, max_chunk)
    assert tr["nc"] == (2 if max_chunk == 20 else 1)
    for t in range(x.shape[0]):
        b = brute.srw_token(x[t].tolist(), h[t].tolist(), e.tolist(), float(tau[t, 0]),
                            r.tolist(), w.tolist(), gate="gelu_v401", onepass=True)
        assert np.allclose(res[0][0, t].numpy(), b["out"], rtol=1e-10, atol=1e-13)
        assert math.isclose(float(tr["den"][0, t, 0]), b["den"], rel_tol=1e-12)
        assert math.isclose(float(tr["tau"][0, t, 0]), b["tau"], rel_tol=1e-11, abs_tol=1e-13)
        assert np.allclose(tr["gate"][0, t].numpy(), b["gates"], rtol=1e-10, atol=1e-15)
        assert int(tr["n_active"][0, t, 0]) == b["n_active"]
        assert b["den"] > 1.0       # the floor is not what the comparison rests on


def test_fused_v401_exact_equals_inference_form():
    """In exact arithmetic the fused function (one-pass std, chunked) and the
    pinned _srw_inference v4.0.1 form (two-pass std, v401:1443-1463) agree."""
    x, h, e, tau, r, w = _v401_inputs(8, T=6, D=16, dr=12, N=90)
    res, _ = _v401_exact(x, h, e, tau, r, w, 30)
    ref = srw_ref.srw_inference_gelu_v401(x, h, e, tau, r, w, acc_dtype=F64)
    assert torch.allclose(res[0][0], ref, rtol=1e-9, atol=1e-13)


def test_fused_v401_diagnostics_closed_forms():
    """The 16-tuple (v401:343-367) against numpy / scipy on the textbook
    float64 score matrix."""
    T, D, dr, N = 24, 32, 16, 300
    x, h, e, tau, r, w = _v401_inputs(9, T=T, D=D, dr=dr, N=N, tau=0.3)
    res, tr = _v401_exact(x, h, e, tau, r, w, 100)
    o = dict(zip(srw_ref.FUSED_V401_OUTPUT_NAMES, res))
    s = (h.numpy() @ e.numpy().T)                                  # [T, N] float64
    mean = s.mean(-1, keepdims=True)
    std = np.sqrt((s * s).mean(-1, keepdims=True) - mean ** 2) + 1e-8
    tau_np = mean + tau.numpy() * std
    z = (s - tau_np) / std
    gate = np.where(z > 0, z * scipy.special.ndtr(z), 0.0)
    act = (z > 0).sum(-1)
    assert np.allclose(tr["gate"][0].numpy(), gate, rtol=1e-10, atol=1e-14)
    assert np.array_equal(np.rint(o["active_frac"][0, :, 0].numpy() * N), act)
    assert np.allclose(o["gate_max"][0, :, 0].numpy(), gate.max(-1), rtol=1e-12)
    z_star = scipy.optimize.brentq(lambda v: v * scipy.special.ndtr(v) - 0.5, 0.0, 3.0)
    assert np.array_equal(np.rint(o["strong_frac"][0, :, 0].numpy() * N), (z > z_star).sum(-1))
    z95 = scipy.special.ndtri(0.95)                                # Phi > .95 <=> z > z95
    assert np.array_equal(np.rint(o["boundary_frac"][0, :, 0].numpy() * N), (np.abs(z) > z95).sum(-1))
    assert np.allclose(o["z_mean_active"][0, :, 0].numpy(),
                       np.where(z > 0, z, 0).sum(-1) / (act + 1e-8), rtol=1e-12)
    assert math.isclose(float(o["tau_abs_mean"]), float(tau_np.mean()), rel_tol=1e-12)
    assert math.isclose(float(o["z_lt_075_frac"]),
                        float((((z > 0) & (z < 0.75)).sum(-1) / (act + 1e-8)).mean()), rel_tol=1e-12)
    assert math.isclose(float(o["z_lt_030_frac"]),
                        float((((z > 0) & (z < 0.30)).sum(-1) / (act + 1e-8)).mean()), rel_tol=1e-12)
    assert math.isclose(float(o["score_std"]), float(std.mean()), rel_tol=1e-12)
    assert math.isclose(float(o["gate_sum"]), float(gate.sum(-1).mean()), rel_tol=1e-12)
    assert math.isclose(float(o["active_n_mean"]), float(act.mean()), rel_tol=1e-12)
    assert math.isclose(float(o["active_per_token_std"]), float(act.std()), rel_tol=1e-12)
    assert math.isclose(float(o["score_skew"]), float(scipy.stats.skew(s, axis=-1).mean()),
                        rel_tol=1e-6, abs_tol=1e-9)
    pn = s.mean(axis=0)
    assert math.isclose(float(o["score_lb"]), float(pn.var() / (pn.mean() ** 2 + pn.var() + 1e-2)),
                        rel_tol=1e-9)
    assert math.isclose(float(o["gate_entropy"]), float(scipy.stats.entropy(gate, axis=-1).mean()),
                        rel_tol=1e-6)


def test_fused_v401_bf16_within_budget_of_exact():
    """The bf16 form (the reference's rounding points) stays within the bf16
    error budget of the exact form; chunking moves only the per-chunk bf16
    rounding of the write GEMM."""
    T, D, dr, N = 32, 64, 32, 900
    x, h, e, tau, r, w = _v401_inputs(10, T=T, D=D, dr=dr, N=N, tau=0.5)
    ex, _ = _v401_exact(x, h, e, tau, r, w, 300)
    bf = srw_ref.fused_gate_srw_gelu_v401(x[None].float(), h[None].float(), e.float(), tau[None].float(),
                                          r.float(), w.float(), max_chunk_size=300)
    rel = float((bf[0][0].double() - ex[0][0]).norm() / ex[0][0].norm())
    assert rel < 1.5e-2
    one = srw_ref.fused_gate_srw_gelu_v401(x[None].float(), h[None].float(), e.float(), tau[None].float(),
                                           r.float(), w.float(), max_chunk_size=4096)
    relc = float((one[0][0] - bf[0][0]).norm() / one[0][0].norm())
    assert 0 < relc < 1e-2


def test_v401_pins_accept_unmutated_oracle():
    assert not _v401_brute_mismatch()


def _gate_gelu_below_zero(raw_f, s_std):
    z = raw_f / s_std
    phi = 0.5 * (1.0 + torch.erf(z * 0.7071067811865476))
    return z, phi, z * phi                    # wrong: no zero for z <= 0


def _gate_gelu_no_sqrt2(raw_f, s_std):
    z = raw_f / s_std
    phi = 0.5 * (1.0 + torch.erf(z))          # wrong: erf(z) for Phi(z)
    return z, phi, torch.where(z > 0, z * phi, torch.zeros((), dtype=z.dtype))


V401_MUTATIONS = {
    "den_from_z_plus_sum": ("_v401_den", lambda g, zp: torch.clamp_min(zp, 1.0)),
    "rows_not_normalised": ("_norm_rows", lambda t: t),
    "gate_below_zero": ("gate_gelu_v401", _gate_gelu_below_zero),
    "phi_without_sqrt2": ("gate_gelu_v401", _gate_gelu_no_sqrt2),
}


@pytest.mark.parametrize("name", sorted(V401_MUTATIONS))
def test_planted_v401_mistakes_are_caught(monkeypatch, name):
    attr, fn = V401_MUTATIONS[name]
    monkeypatch.setattr(srw_ref, attr, fn)
    assert _v401_brute_mismatch()


# ---------------------------------------------------------------- gate_norm

def _gate_norm_matches_brute(gate_norm, x, h, e, tau, r, w):
    """gate_norm (v41:1760) against gate / max(sum gate, 1e-8) of the
    brute-force loop's gates."""
    for t in range(x.shape[0]):
        b = brute.srw_token(x[t].tolist(), h[t].tolist(), e.tolist(), float(tau[t, 0]),
                            r.tolist(), w.tolist())
        g = np.array(b["gates"])
        if not np.allclose(gate_norm[t].numpy(), g / max(g.sum(), 1e-8), rtol=1e-10, atol=1e-300):
            return False
    return True


def test_gate_norm_matches_brute_force_and_sums_to_one():
    T, D, dr, N = 4, 12, 8, 40
    x, h, e, tau, r, w = _rand_inputs(T, D, dr, N, 21)
    out, gate, gnorm = srw_ref.srw_inference_with_gates(x, h, e, tau, r, w, acc_dtype=F64)
    assert _gate_norm_matches_brute(gnorm, x, h, e, tau, r, w)
    assert torch.allclose(gnorm.sum(-1), torch.ones(T, dtype=F64), rtol=1e-12)
    assert torch.equal(out, srw_ref.srw_inference(x, h, e, tau, r, w, acc_dtype=F64))
    # plausible mistakes fail the same check
    _, tr = srw_ref.srw_inference(x, h, e, tau, r, w, acc_dtype=F64, return_trace=True)
    assert not _gate_norm_matches_brute(gate / tr["intensity"].sum(-1, keepdim=True), x, h, e, tau, r, w)
    assert not _gate_norm_matches_brute(gate / tr["den"], x, h, e, tau, r, w)
    assert not _gate_norm_matches_brute(tr["activation"] / tr["activation"].sum(-1, keepdim=True),
                                        x, h, e, tau, r, w)


def test_gate_norm_floor():
    """Every margin well below zero: sum gate < 1e-8, so gate_norm = gate / 1e-8
    (the clamp of v41:1760), not gate / sum gate."""
    T, D, dr, N = 3, 12, 8, 40
    x, h, e, tau, r, w = _rand_inputs(T, D, dr, N, 22, tau=2.4)
    _, gate, gnorm = srw_ref.srw_inference_with_gates(x, h, e, tau, r, w, acc_dtype=F64)
    assert bool((gate.sum(-1) < 1e-8).all()) and bool((gate.sum(-1) > 0).all())
    assert torch.equal(gnorm, gate / 1e-8)
    assert _gate_norm_matches_brute(gnorm, x, h, e, tau, r, w)
    assert not _gate_norm_matches_brute(gate / gate.sum(-1, keepdim=True), x, h, e, tau, r, w)


# ---------------------------------------------------------------- v4.0.1 paired function
#
# fused_gate_srw_gelu_v401_paired (v401:408-554) against ONE single-route call
# (fused_gate_srw_gelu_v401, pinned above against brute force, closed forms and
# scipy) over the 2*B*S virtual rows (token t, route r) -> row (s, r) of a
# [B, 2S] batch with x repeated per route, in exact arithmetic: every statistic
# of the paired function is per (token, route) row over N (v401:426-457), so
# that single call holds every row of it, and its reductions fix the paired
# ones -- out route by route (den per route, v401:521-524); the active / gate
# max / strong / boundary fractions and z_mean_active as route means
# (v401:525-538); every scalar over (B, S, 2), score_lb from per-unit means
# over (B, S, 2) (v401:436).

_V401_PAIRED_ROUTE_MEAN = ("active_frac", "gate_max", "strong_frac", "boundary_frac", "z_mean_active")


def _v401_paired_vs_single_mismatch(seed=23):
    B, S, D, dr, N = 2, 6, 24, 16, 360
    x, h, e, tau, r, w = _v401_inputs(seed, T=B * S, D=D, dr=dr, N=N, tau=0.1)
    g = torch.Generator().manual_seed(seed + 1)
    h2 = torch.stack([h, torch.randn(B * S, dr, generator=g, dtype=F64)], dim=1)   # [T, 2, dr]
    tau2 = torch.stack([tau, tau + 0.4], dim=1)                                   # [T, 2, 1]
    pr = srw_ref.fused_gate_srw_gelu_v401_paired(x.reshape(B, S, D), h2.reshape(B, S, 2, dr), e,
                                                 tau2.reshape(B, S, 2, 1), r, w, max_chunk_size=90,
                                                 exact=True)
    xs = x.reshape(B, S, 1, D).expand(B, S, 2, D).reshape(B, 2 * S, D)
    sg = srw_ref.fused_gate_srw_gelu_v401(xs, h2.reshape(B, 2 * S, dr), e, tau2.reshape(B, 2 * S, 1), r, w,
                                          max_chunk_size=90, exact=True)
    P = dict(zip(srw_ref.FUSED_V401_OUTPUT_NAMES, pr))
    Q = dict(zip(srw_ref.FUSED_V401_OUTPUT_NAMES, sg))
    bad = []
    for name in srw_ref.FUSED_V401_OUTPUT_NAMES:
        p, q = P[name], Q[name]
        if name == "out":
            q = q.reshape(B, S, 2, D)
        elif name in _V401_PAIRED_ROUTE_MEAN:
            q = q.reshape(B, S, 2, 1).mean(dim=2)
        if p.shape != q.shape or not torch.allclose(p, q, rtol=1e-10, atol=1e-12):
            bad.append(name)
    return bad


def test_v401_paired_equals_one_single_over_route_rows():
    assert _v401_paired_vs_single_mismatch() == []


V401_PAIRED_MUTATIONS = {
    # per-unit score means per route (over (B, S) only) for score_lb
    "score_lb_per_route": ("_unit_means", lambda s, axes: s.mean(dim=axes[:2]), "score_lb"),
    # per-token fractions of route 0 instead of the route mean
    "active_frac_unaveraged": ("_route_mean", lambda t: t[:, :, 0], "active_frac"),
    # one den for both routes (the routes' gate sums added)
    "den_over_routes": ("_v401_den", lambda g, zp: torch.clamp_min(g.sum(dim=-2, keepdim=True), 1.0), "out"),
}


@pytest.mark.parametrize("name", sorted(V401_PAIRED_MUTATIONS))
def test_planted_v401_paired_mistakes_are_caught(monkeypatch, name):
    attr, fn, field = V401_PAIRED_MUTATIONS[name]
    monkeypatch.setattr(srw_ref, attr, fn)
    assert field in _v401_paired_vs_single_mismatch()


def test_v401_autograd_matches_finite_differences():
    """The GPU backward of the v4.0.1 gate is checked against torch autograd
    through fused_gate_srw_gelu_v401; in exact arithmetic that autograd
    equals central finite differences of <d_out, out> + d_lb score_lb in
    every input (x, h, emb, tau_offset, read, write)."""
    T, D, dr, N = 10, 12, 8, 48
    x, h, e, tau, r, w = _v401_inputs(31, T=T, D=D, dr=dr, N=N, tau=0.2)
    g = torch.Generator().manual_seed(32)
    d_out = torch.randn(T, D, generator=g, dtype=F64)

    def loss(*a):
        res = srw_ref.fused_gate_srw_gelu_v401(a[0][None], a[1][None], a[2], a[3][None], a[4], a[5],
                                               max_chunk_size=16, exact=True)
        return (res[0][0] * d_out).sum() + 0.37 * res[3]

    inputs = [x, h, e, tau, r, w]
    leaves = [t.clone().requires_grad_(True) for t in inputs]
    loss(*leaves).backward()
    eps = 1e-6
    for i, t in enumerate(inputs):
        for (a, b) in ((0, 0), (t.shape[0] // 2, t.shape[1] - 1), (t.shape[0] - 1, t.shape[1] // 2)):
            p = [u.clone() for u in inputs]
            m = [u.clone() for u in inputs]
            p[i][a, b] += eps
            m[i][a, b] -= eps
            fd = float((loss(*p) - loss(*m)) / (2 * eps))
            assert math.isclose(float(leaves[i].grad[a, b]), fd, rel_tol=1e-5, abs_tol=1e-8), (i, a, b)
