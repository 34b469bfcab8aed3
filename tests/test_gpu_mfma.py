"""GPU parity of the matrix-core paths (libsrw_amd.so's fused "mfma_bf16"
kernels and the "tiled_bf16" GEMM family, through the C ABI) against the CPU
oracle's restatement of fused_gate_srw (models/dawn_spatial_v41_exp.py:415-635).

Shapes cover: d_route == d_model with h aliasing x (the Know-pool form of
the benchmark), a separate router h with d_route = 128, ragged N (not a
multiple of the 32-unit tile), ragged T (not a multiple of the 128-token
tile), reference chunk boundaries that fall inside a unit tile, the den
floor, and the full configs[0] size.

Tolerances: out within 2e-2 relative (Frobenius) of the bf16 restatement,
and the passing set identical outside a tie band of one bf16 score ulp plus
the tau slack -- the score GEMM's fp32 accumulation order differs from the
CPU matmul, so a score can round to the neighbouring bf16 value -- with the
count inside the band bounded (tests/parity.py).
"""

from __future__ import annotations

import pytest
import torch

from oracle import srw_ref
from tests.parity import (REL_BF16, assert_pass_set, bf16_ulp, rel_fro, row_rel_max,
                          unpack_mask)

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


def _inputs(pkg, T, D, dr, N, h_is_x, seed, tau=-0.5):
    shape = pkg.inputs.PoolShape(T=T, D=D, N=N, dr=dr, routes=1, h_is_x=h_is_x)
    inp = pkg.inputs.make_pool_inputs(shape, seed=seed)
    inp["tau_offset"].fill_(tau)
    return inp


# the fused family: the main kernel that recomputes the scores, the one that
# streams the moments kernel's scores (d_route >= d_model), and the decode
# kernel for calls of at most 128 rows
FUSED = ("mfma_bf16", "mfma_ss_bf16", "mfma_decode_bf16")
FAMILIES = {"fused": (FUSED, {}), "tiled": (("tiled_bf16",), {"tiled": True})}


def _gpu(pkg, dev, inp, chunk_size, **kw):
    x = inp["x"].to(BF).to(dev)
    h = x if "h" not in inp else inp["h"].to(BF).to(dev)
    res = pkg.srw_forward(x, h, inp["emb"].to(BF).to(dev), inp["tau_offset"].to(dev),
                          inp["read"].to(BF).to(dev), inp["write"].to(BF).to(dev),
                          chunk_size=chunk_size, **kw)
    torch.cuda.synchronize()
    return {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in res.items()}


def _oracle(inp, max_chunk):
    x = inp["x"][None]
    h = x if "h" not in inp else inp["h"][:, 0][None]
    return srw_ref.fused_gate_srw(x, h, inp["emb"], inp["tau_offset"][None], inp["read"],
                                  inp["write"], max_chunk_size=max_chunk, return_trace=True)


def _gram_delta(inp, tr):
    """Gram moments are those of the unrounded scores: the tie band widens by
    |tau(unrounded scores) - tau(bf16 scores)|, computed here in fp64."""
    T = inp["x"].shape[0]
    h = inp["x"] if "h" not in inp else inp["h"][:, 0]
    s64 = h.to(torch.bfloat16).double() @ inp["emb"].to(torch.bfloat16).double().T
    mean = s64.mean(dim=1)
    std = torch.sqrt((s64 * s64).mean(dim=1) - mean * mean) + 1e-8
    tau_g = mean + inp["tau_offset"][:, 0].double() * std
    dtau = (tau_g - tr["tau"].reshape(T).double()).abs().float()
    print(f"  max |tau_gram - tau_ref| = {float(dtau.max()):.2e}", flush=True)
    return 2 * dtau + 1e-6


def _check(got, ref, tr, T, N, D, out_tol=REL_BF16, extra_delta=None):
    out_ref = ref[0].reshape(T, D)
    out = got["out"][:, 0].float()
    err = rel_fro(out, out_ref)
    print(f"  out rel err {err:.3e}, worst row {row_rel_max(out, out_ref):.3e}", flush=True)
    assert err <= out_tol
    assert row_rel_max(out, out_ref) <= 5e-2
    den_ref = tr["den"].reshape(T)
    den_tol = 2e-4 * den_ref
    if extra_delta is not None:
        # a tau shift moves every active unit's intensity by the same amount
        den_tol = den_tol + tr["n_active"].reshape(T) * extra_delta.reshape(T)
    assert bool(((got["den"][:, 0] - den_ref).abs() <= den_tol).all())
    assert torch.allclose(got["gate_sum"][:, 0], tr["gate_sum"].reshape(T), rtol=2e-3, atol=1e-5)
    margin = tr["margin"].reshape(T, N)
    score = margin + tr["tau"].reshape(T, 1) + 0.5
    # one bf16 ulp of the score + a bound on the moments' fp32 summation
    # difference in tau
    delta = bf16_ulp(score) + 1e-4 * tr["s_std"].reshape(T, 1)
    mask = unpack_mask(got["pass_mask"][:, 0], N)
    assert_pass_set(mask, margin, delta,
                    shift=None if extra_delta is None else extra_delta.reshape(T, 1).expand(T, N))
    # bits beyond N in the last word are zero
    words = got["pass_mask"][:, 0]
    full = unpack_mask(words, words.shape[-1] * 64)
    assert not bool(full[:, N:].any())
    # n_active is the popcount of the mask
    assert torch.equal(got["n_active"][:, 0].long(), mask.sum(dim=1))


CASES = [
    # T, D, dr, N, h_is_x, max_chunk (reference), seed
    (256, 384, 384, 2600, True, 1300, 1),     # chunk boundary 1300 inside a tile
    (200, 384, 128, 1580, False, 12500, 2),   # ragged T and N, router h
    (77, 128, 64, 777, False, 300, 3),        # three chunks of 259 units
    (33, 64, 64, 100, True, 2048, 4),         # tiny pool, one chunk
    (130, 128, 128, 70, True, 2048, 5),       # odd tile count: upper half of last word unused
]


@pytest.mark.parametrize("family", sorted(FAMILIES))
@pytest.mark.parametrize("case", CASES, ids=lambda c: "T{}D{}dr{}N{}{}c{}".format(
    c[0], c[1], c[2], c[3], "x" if c[4] else "", c[5]))
def test_mfma_matches_fused_oracle(pkg, dev, case, family):
    T, D, dr, N, hx, max_chunk, seed = case
    print(f"[gpu] {family} bf16 {case}", flush=True)
    inp = _inputs(pkg, T, D, dr, N, hx, seed)
    _, cs = srw_ref.chunk_plan(N, max_chunk)
    path, kw = FAMILIES[family]
    got = _gpu(pkg, dev, inp, cs, **kw)
    assert got["path"] in path
    ref, tr = _oracle(inp, max_chunk)
    _check(got, ref, tr, T, N, D)


@pytest.mark.parametrize("case", [
    (256, 384, 384, 2600, True, 1300, 21),    # chunk boundary inside a tile, h aliases x
    (300, 128, 128, 1580, False, 12500, 22),  # ragged last token tile, router h
    (200, 128, 128, 777, False, 300, 23),     # three chunks
    (33, 64, 64, 100, True, 2048, 24),        # d_model 64, one partial tile
], ids=lambda c: "T{}D{}dr{}N{}{}c{}".format(c[0], c[1], c[2], c[3], "x" if c[4] else "", c[5]))
def test_mfma_streamed_scores_diag_split_equals_plain(pkg, dev, case):
    """With d_route >= d_model the fused forward's main kernel reads back the
    bf16 scores the moments kernel stored (srw_main_ss_kernel).  With
    diagnostics its producer waves take the intensity sum, pass bits and
    active count of the tile the consumers gate (from the same LDS score
    stage) while the consumers keep the gate sum: the same scores, tau and
    element order, so the layer outputs are equal bit for bit to the call
    without diagnostics.  (The diagnostics themselves are checked against the
    scalar kernels in test_mfma_diagnostics_match_generic.)"""
    T, D, dr, N, hx, max_chunk, seed = case
    print(f"[gpu] streamed scores, diagnostics on and off {case}", flush=True)
    inp = _inputs(pkg, T, D, dr, N, hx, seed)
    inp["tau_offset"].uniform_(-0.9, 0.6, generator=torch.Generator().manual_seed(seed))
    _, cs = srw_ref.chunk_plan(N, max_chunk)
    a = _gpu(pkg, dev, inp, cs)
    b = _gpu(pkg, dev, inp, cs, diag=True)
    assert a["path"] == b["path"] == "mfma_ss_bf16"
    for k in ("out", "den", "gate_sum", "n_active", "pass_mask"):
        assert torch.equal(a[k], b[k]), k


GRAM_CASES = [
    (256, 384, 384, 2600, True, 1300, 11),
    (200, 384, 128, 1580, False, 12500, 12),
    (77, 128, 64, 777, False, 300, 13),
    (64, 64, 32, 100, False, 2048, 14),
]


@pytest.mark.parametrize("case", GRAM_CASES, ids=lambda c: "T{}D{}dr{}N{}{}c{}".format(
    c[0], c[1], c[2], c[3], "x" if c[4] else "", c[5]))
def test_mfma_gram_stats_matches_fused_oracle(pkg, dev, case):
    """Moments from G = E^T E and sum e (SRW_STATS_GRAM) instead of the score
    pre-pass: same output and passing-set bar as the one-pass path."""
    T, D, dr, N, hx, max_chunk, seed = case
    print(f"[gpu] mfma bf16 gram {case}", flush=True)
    inp = _inputs(pkg, T, D, dr, N, hx, seed)
    _, cs = srw_ref.chunk_plan(N, max_chunk)
    got = _gpu(pkg, dev, inp, cs, stats="gram")
    assert got["path"] in FUSED
    ref, tr = _oracle(inp, max_chunk)
    _check(got, ref, tr, T, N, D, extra_delta=_gram_delta(inp, tr))


def test_mfma_gram_equals_onepass_closely(pkg, dev):
    """Gram moments vs the bf16-score pre-pass on the same inputs: den and the
    outputs agree to well inside the bf16 tolerance."""
    T, D, dr, N = 512, 384, 384, 6000
    print(f"[gpu] gram vs onepass T{T} N{N}", flush=True)
    inp = _inputs(pkg, T, D, dr, N, True, seed=17)
    a = _gpu(pkg, dev, inp, 0, stats="onepass")
    b = _gpu(pkg, dev, inp, 0, stats="gram")
    assert rel_fro(b["out"].float(), a["out"].float()) <= 2e-3
    assert torch.allclose(b["den"], a["den"], rtol=1e-3)  # n_active * |d tau| / den ~ 1e-4
    mism = (unpack_mask(a["pass_mask"][:, 0], N) != unpack_mask(b["pass_mask"][:, 0], N)).sum()
    assert int(mism) <= T * N * 1e-4


CENTERED_CASES = [
    # T, D, dr, N, h_is_x, seed
    (256, 384, 384, 2600, True, 31),    # Know-pool form, ragged N
    (200, 384, 128, 1580, False, 32),   # router h, ragged T and N
    (33, 64, 64, 100, True, 33),        # tiny pool
    (130, 128, 128, 70, True, 34),      # a single partial tile per row
]


@pytest.mark.parametrize("family", sorted(FAMILIES))
@pytest.mark.parametrize("case", CENTERED_CASES, ids=lambda c: "T{}D{}dr{}N{}{}".format(
    c[0], c[1], c[2], c[3], "x" if c[4] else ""))
def test_mfma_centered_matches_srw_inference_oracle(pkg, dev, case, family):
    """bf16 _srw_inference (v41:1713-1738) on the matrix cores: the two-pass
    centred std (:1719-1721) from a second moments pass over the same bf16
    scores, one unchunked write GEMM rounded once.  Same bar as the fused
    path: out, den, gate sum and the passing set against the oracle; a tail
    tile that counted padded units as deviations of -mean would move den."""
    T, D, dr, N, hx, seed = case
    print(f"[gpu] {family} bf16 centered {case}", flush=True)
    inp = _inputs(pkg, T, D, dr, N, hx, seed)
    path, kw = FAMILIES[family]
    got = _gpu(pkg, dev, inp, 0, stats="centered", **kw)
    assert got["path"] in path
    x = inp["x"].to(BF)
    h = x if "h" not in inp else inp["h"][:, 0].to(BF)
    ref, tr = srw_ref.srw_inference(x, h, inp["emb"].to(BF), inp["tau_offset"], inp["read"].to(BF),
                                    inp["write"].to(BF), return_trace=True)
    raw = tr["scores"] - tr["tau"]
    flat = dict(margin=raw - 0.5, tau=tr["tau"], s_std=tr["s_std"], den=tr["den"],
                gate_sum=tr["gate"].sum(dim=-1), n_active=(tr["activation"] > 0.5).sum(dim=-1))
    _check(got, (ref,), flat, T, N, D)
    # the generic kernels' centred sweep: same fp32 two-pass sums in another order
    gen = _gpu(pkg, dev, inp, 0, stats="centered", force_generic=True)
    assert gen["path"] == "generic"
    assert torch.allclose(got["den"], gen["den"], rtol=1e-4)
    assert rel_fro(got["out"].float(), gen["out"].float()) <= 1e-2


PAIRED_CASES = [
    # T, D, dr, N, max_chunk, seed
    (128, 384, 128, 1580, 12500, 21),   # the 40M QK pool with the router's d_route
    (100, 384, 384, 700, 12500, 22),    # configs[1] d_route = d_model, ragged T and N
    (70, 128, 64, 777, 300, 23),        # three reference chunks
]


@pytest.mark.parametrize("family", sorted(FAMILIES))
@pytest.mark.parametrize("case", PAIRED_CASES, ids=lambda c: "T{}D{}dr{}N{}c{}".format(*c[:5]))
def test_mfma_paired_matches_fused_paired_oracle(pkg, dev, case, family):
    """Paired QK routes (fused_gate_srw_paired, v41:640-909) on the matrix cores."""
    T, D, dr, N, max_chunk, seed = case
    print(f"[gpu] {family} bf16 paired {case}", flush=True)
    shape = pkg.inputs.PoolShape(T=T, D=D, N=N, dr=dr, routes=2)
    inp = pkg.inputs.make_pool_inputs(shape, seed=seed)
    _, cs = srw_ref.chunk_plan(N, max_chunk)
    path, kw = FAMILIES[family]
    got = _gpu(pkg, dev, inp, cs, **kw)
    assert got["path"] in path
    ref, tr = srw_ref.fused_gate_srw_paired(
        inp["x"][None], inp["h"][None], inp["emb"], inp["tau_offset"].reshape(1, T, 2, 1),
        inp["read"], inp["write"], max_chunk_size=max_chunk, return_trace=True)
    # rows are (token, route) pairs: check them as 2T single-route rows
    flat = dict(margin=tr["margin"].reshape(2 * T, N), tau=tr["tau"].reshape(2 * T, 1),
                s_std=tr["s_std"].reshape(2 * T, 1), den=tr["den"].reshape(2 * T),
                gate_sum=tr["gate_sum"].reshape(2 * T), n_active=tr["n_active"].reshape(2 * T))
    got2 = {k: (v.reshape(2 * T, *v.shape[2:]) if isinstance(v, torch.Tensor) and v.dim() >= 2
                and v.shape[:2] == (T, 2) else v) for k, v in got.items()}
    got2 = {k: (v[:, None] if isinstance(v, torch.Tensor) and k in ("out", "gate_sum", "den",
                                                                     "n_active", "pass_mask") else v)
            for k, v in got2.items()}
    _check(got2, (ref[0].reshape(2 * T, D),), flat, 2 * T, N, D)


def test_mfma_paired_equals_two_singles(pkg, dev):
    """paired(Q, K) == (single(Q), single(K)) on the same pool (v41:796-797)."""
    T, D, dr, N = 96, 384, 128, 1580
    print(f"[gpu] paired vs two singles T{T} N{N}", flush=True)
    shape = pkg.inputs.PoolShape(T=T, D=D, N=N, dr=dr, routes=2)
    inp = pkg.inputs.make_pool_inputs(shape, seed=31)
    both = _gpu(pkg, dev, inp, 0)
    for r in range(2):
        one = dict(inp, h=inp["h"][:, r:r + 1].contiguous(), tau_offset=inp["tau_offset"][:, r:r + 1].contiguous())
        single = _gpu(pkg, dev, one, 0)
        assert single["path"] in FUSED
        assert rel_fro(both["out"][:, r].float(), single["out"][:, 0].float()) <= 1e-3
        # different N-split geometry -> fp32 summation order differs; only
        # units within rounding of the threshold may flip
        mism = (unpack_mask(both["pass_mask"][:, r], N) != unpack_mask(single["pass_mask"][:, 0], N)).sum()
        assert int(mism) <= 4
        assert torch.allclose(both["den"][:, r], single["den"][:, 0], rtol=1e-5)


def test_mfma_den_floor(pkg, dev):
    """A high tau_offset on a V-sized pool: sum intensity < 1, den floors at 1."""
    T, D, dr, N = 64, 384, 384, 2600
    print(f"[gpu] mfma den floor T{T} N{N}", flush=True)
    inp = _inputs(pkg, T, D, dr, N, True, seed=21, tau=3.0)
    got = _gpu(pkg, dev, inp, 0)
    assert got["path"] in FUSED
    ref, tr = _oracle(inp, 12500)
    assert (tr["intensity_sum"] < 1).any()
    assert torch.equal(got["den"][:, 0] == 1.0, tr["den"].reshape(T) == 1.0)
    _check(got, ref, tr, T, N, D)


def test_mfma_matches_generic_kernel(pkg, dev):
    """The matrix-core path against the bit-faithful scalar kernels on the GPU."""
    T, D, dr, N = 512, 384, 384, 6000
    print(f"[gpu] mfma vs generic T{T} N{N}", flush=True)
    inp = _inputs(pkg, T, D, dr, N, True, seed=7)
    _, cs = srw_ref.chunk_plan(N, 2500)
    fast = _gpu(pkg, dev, inp, cs)
    slow = _gpu(pkg, dev, inp, cs, emulate=True)
    assert fast["path"] in FUSED and slow["path"] == "generic"
    assert rel_fro(fast["out"].float(), slow["out"].float()) <= 5e-3
    assert torch.allclose(fast["den"], slow["den"], rtol=2e-4)


def test_mfma_full_know_config(pkg, dev):
    """configs[0] at full size: T=4096, D=384, N=25200, two reference chunks."""
    shape = pkg.inputs.CONFIGS["know"]
    print(f"[gpu] mfma full Know config {shape}", flush=True)
    inp = pkg.inputs.make_pool_inputs(shape, seed=0)
    _, cs = srw_ref.chunk_plan(shape.N, 12500)
    got = _gpu(pkg, dev, inp, cs)
    assert got["path"] in FUSED
    # the oracle on a token subset (rows are independent across tokens)
    Ts = 512
    sub = dict(inp, x=inp["x"][:Ts], tau_offset=inp["tau_offset"][:Ts])
    ref, tr = _oracle(sub, 12500)
    got_s = {k: (v[:Ts] if isinstance(v, torch.Tensor) and v.shape[0] == shape.T else v)
             for k, v in got.items()}
    _check(got_s, ref, tr, Ts, shape.N, shape.D)
    # whole-batch properties: about half the units pass (tau_offset = -0.5),
    # den = N eps + sum_{margin > cutoff} min(margin - cutoff, 10) >= N eps
    frac = got["n_active"].float().mean().item() / shape.N
    assert 0.45 < frac < 0.55, frac
    assert bool((got["den"] >= shape.N * 1e-4).all())
    assert bool(torch.isfinite(got["out"].float()).all())


@pytest.mark.parametrize("stats", ["onepass", "gram"])
def test_mfma_pool_cached_reuses_pool_data(pkg, dev, stats):
    """Decode-style steps over one pool: a plan launched once, then fed new
    tokens in place and launched with pool_cached=True (packed W^T and Gram
    statistics reused from the workspace), gives exactly what a fresh call
    on the new tokens gives."""
    T, D, dr, N = 64, 384, 384, 6100
    print(f"[gpu] mfma pool cached {stats} T{T} N{N}", flush=True)
    _, cs = srw_ref.chunk_plan(N, 2500)
    a = _inputs(pkg, T, D, dr, N, True, seed=31)
    b = _inputs(pkg, T, D, dr, N, True, seed=32)
    b.update(emb=a["emb"], read=a["read"], write=a["write"])
    b["tau_offset"].uniform_(-0.8, 0.2)
    x = a["x"].to(BF).to(dev)
    plan = pkg.SrwPlan(x, x, a["emb"].to(BF).to(dev), a["tau_offset"].to(dev),
                       a["read"].to(BF).to(dev), a["write"].to(BF).to(dev), stats=stats,
                       chunk_size=cs)
    plan.launch()
    first = plan.out.clone()
    plan.inputs[0].copy_(b["x"].to(BF))
    plan.inputs[3].copy_(b["tau_offset"])
    plan.launch(pool_cached=True)
    torch.cuda.synchronize()
    assert plan.path in FUSED
    fresh = _gpu(pkg, dev, b, cs, stats=stats)
    assert torch.equal(plan.out.cpu(), fresh["out"])
    assert torch.equal(plan.den.cpu(), fresh["den"])
    assert torch.equal(plan.pass_mask.cpu(), fresh["pass_mask"])
    assert not torch.equal(first.cpu(), fresh["out"])
    ref, tr = _oracle(b, 2500)
    _check(fresh, ref, tr, T, N, D, extra_delta=_gram_delta(b, tr) if stats == "gram" else None)


def _diag_scores(inp, hx, R):
    """bf16 scores [T, R, N] as the reference rounds them (v41:439)."""
    T = inp["x"].shape[0]
    h = inp["x"][:, None] if hx else inp["h"]
    s = h.to(torch.bfloat16).float() @ inp["emb"].to(torch.bfloat16).float().T
    return s.to(torch.bfloat16).float().reshape(T, R, -1)


DIAG_CASES = [
    # T, D, dr, N, h_is_x, routes, max_chunk, seed
    (256, 384, 384, 6000, True, 1, 2500, 41),   # Know form, two reference chunks
    (200, 384, 128, 1580, False, 2, 12500, 42),  # paired QK pool with the router's d_route
    (130, 128, 64, 1000, False, 1, 300, 43),    # four chunks, ragged T
    (300, 128, 128, 1580, False, 1, 700, 44),   # streamed scores with the router's h, chunk edge in a tile
]


@pytest.mark.parametrize("case", DIAG_CASES, ids=lambda c: "T{}D{}dr{}N{}R{}".format(c[0], c[1], c[2], c[3], c[5]))
def test_mfma_diagnostics_match_generic(pkg, dev, case):
    """SRW_FLAG_DIAG on the matrix-core path: token_diag [T,R,14] and
    unit_diag [N,2] against the reference-faithful scalar kernels
    (v41:442-552).  Band counts use thresholds on the exp argument (the exact
    inverse of the act thresholds), so elements within rounding of a band edge
    may fall on the other side: counts agree to 2 + 1e-3 N."""
    T, D, dr, N, hx, R, max_chunk, seed = case
    print(f"[gpu] mfma diagnostics {case}", flush=True)
    shape = pkg.inputs.PoolShape(T=T, D=D, N=N, dr=dr, routes=R, h_is_x=hx)
    inp = pkg.inputs.make_pool_inputs(shape, seed=seed)
    inp["tau_offset"].uniform_(-0.9, 0.3, generator=torch.Generator().manual_seed(seed))
    _, cs = srw_ref.chunk_plan(N, max_chunk)
    x = inp["x"].to(BF).to(dev)
    h = x if hx else inp["h"].to(BF).to(dev)
    args = (x, h, inp["emb"].to(BF).to(dev), inp["tau_offset"].to(dev), inp["read"].to(BF).to(dev),
            inp["write"].to(BF).to(dev))
    fast = pkg.srw_forward(*args, chunk_size=cs, diag=True)
    slow = pkg.srw_forward(*args, chunk_size=cs, diag=True, emulate=True)
    torch.cuda.synchronize()
    assert fast["path"] in FUSED and slow["path"] == "generic"
    f = {k: v.cpu() for k, v in fast.items() if isinstance(v, torch.Tensor)}
    g = {k: v.cpu() for k, v in slow.items() if isinstance(v, torch.Tensor)}
    assert rel_fro(f["out"].float(), g["out"].float()) <= 5e-3
    assert torch.allclose(f["den"], g["den"], rtol=2e-4)
    td_f, td_g = f["token_diag"], g["token_diag"]
    names = ["s_mean", "s_std", "tau", "sum_s3", "sum_s4", "gate_max", "int_sum", "n_strong",
             "n_boundary", "n_band075", "n_band030", "g_log_g", "int_max", "n_int_cap"]
    col = {n: i for i, n in enumerate(names)}
    for n in ("s_mean", "s_std", "tau"):
        assert torch.allclose(td_f[..., col[n]], td_g[..., col[n]], rtol=1e-4, atol=1e-5), n
    # power sums of the bf16 scores: the two paths accumulate each score in a
    # different fp32 order, so a score can round to the neighbouring bf16
    # value (about 1 in 10^3 near a rounding midpoint); bound the deviation by
    # a fraction of sum_n k |s|^(k-1) ulp(s) computed from the oracle's scores
    sc = _diag_scores(inp, hx, R)
    for k, n in ((3, "sum_s3"), (4, "sum_s4")):
        sens = (k * sc.abs() ** (k - 1) * bf16_ulp(sc)).sum(dim=-1).reshape(td_g[..., 0].shape)
        d = (td_f[..., col[n]] - td_g[..., col[n]]).abs()
        bound = 0.02 * sens + 1e-5 * (sc.abs() ** k).sum(dim=-1).reshape(d.shape)
        print(f"  {n}: max |diff| {float(d.max()):.3e}, max diff/bound {float((d / bound).max()):.3f}", flush=True)
        assert (d <= bound).all(), n
    for n in ("gate_max", "int_max", "int_sum"):
        assert torch.allclose(td_f[..., col[n]], td_g[..., col[n]], rtol=2e-3, atol=1e-6), n
    # sum g log g mixes positive (g > 1) and negative terms and may cancel:
    # bound the difference by the sum of the terms' magnitudes (v4.1 gate of
    # the oracle's bf16 scores and the generic kernel's tau)
    m = sc - td_g[..., col["tau"]][..., None] - 0.5
    gt = torch.sigmoid(500.0 * m) * (1e-4 + torch.clamp(m - 0.01, 0.0, 10.0))
    mag = (gt * torch.log(gt + 1e-8)).abs().sum(dim=-1)
    d = (td_f[..., col["g_log_g"]] - td_g[..., col["g_log_g"]]).abs()
    bound = 1e-3 + 2e-3 * td_g[..., col["g_log_g"]].abs() + 1e-4 * mag
    print(f"  g_log_g: max |diff| {float(d.max()):.3e}, max diff/bound {float((d / bound).max()):.3f}", flush=True)
    assert (d <= bound).all(), "g_log_g"
    for n in ("n_strong", "n_boundary", "n_band075", "n_band030", "n_int_cap"):
        d = (td_f[..., col[n]] - td_g[..., col[n]]).abs()
        print(f"  {n}: max |diff| {float(d.max())}", flush=True)
        assert (d <= 2 + 1e-3 * N).all(), n
    ud_f, ud_g = f["unit_diag"], g["unit_diag"]
    assert torch.allclose(ud_f[:, 0], ud_g[:, 0], rtol=1e-3, atol=1e-3 * (T * R) ** 0.5), "score_sum"
    assert torch.allclose(ud_f[:, 1], ud_g[:, 1], rtol=2e-3, atol=1e-6), "unit gate_max"
    assert torch.equal(f["n_active"], g["n_active"]) or int((f["n_active"] - g["n_active"]).abs().max()) <= 2


def test_mfma_graph_replay_matches_eager(pkg, dev):
    """One call captured in a HIP graph and replayed three times, with eager
    work between the replays (new tokens copied in place): every replay
    equals an eager call on the same inputs.  With diagnostics, so the
    unit_diag clear (a fill kernel, no memset node) and its atomics replay
    too; the atomic per-unit score sums may differ in the last bits."""
    T, D, dr, N = 256, 384, 128, 3000
    print(f"[gpu] mfma graph replay T{T} D{D} dr{dr} N{N}", flush=True)
    shape = pkg.inputs.PoolShape(T=T, D=D, N=N, dr=dr, routes=1, h_is_x=False)
    inp = pkg.inputs.make_pool_inputs(shape, seed=51)
    bf = BF
    plan = pkg.SrwPlan(inp["x"].to(bf).to(dev), inp["h"].to(bf).to(dev), inp["emb"].to(bf).to(dev),
                       inp["tau_offset"].to(dev), inp["read"].to(bf).to(dev),
                       inp["write"].to(bf).to(dev), chunk_size=1500, diag=True)
    plan.launch()
    torch.cuda.synchronize()
    assert plan.path in FUSED
    cur = torch.cuda.current_stream(dev)
    cap = torch.cuda.Stream(dev)
    cap.wait_stream(cur)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=cap):
        plan.launch(cap)
    torch.cuda.synchronize()
    gen = torch.Generator().manual_seed(52)
    keys = ("out", "gate_sum", "den", "n_active", "pass_mask", "token_diag")
    for rep in range(3):
        plan.inputs[0].copy_(torch.randn(T, D, generator=gen).to(bf))
        plan.inputs[1].copy_(torch.randn(T, 1, dr, generator=gen).to(bf))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = {k: plan.results()[k].clone() for k in keys + ("unit_diag",)}
        plan.launch()
        torch.cuda.synchronize()
        ref = plan.results()
        for k in keys:
            assert torch.equal(got[k], ref[k]), (rep, k)
        assert torch.equal(got["unit_diag"][:, 1], ref["unit_diag"][:, 1]), rep
        assert torch.allclose(got["unit_diag"][:, 0], ref["unit_diag"][:, 0], rtol=1e-5, atol=1e-4), rep
