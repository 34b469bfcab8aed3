"""GPU parity of the v4.0.1 GELU gate on the matrix-core kernels (the
recomputing main kernel and the decode kernel, through the C ABI) against
the oracle's ``fused_gate_srw_gelu_v401`` (models/legacy/dawn_spatial_v401_exp.py:230-367)
and ``srw_inference_gelu_v401`` (v401:1443-1463), both pinned on the CPU
(tests/test_oracle_pins.py).

The kernels forward-normalise the read and write rows in bf16 (v401:300-301),
gate with z Phi(z) for z = (s - tau) / s_std > 0 (v401:303-306; Phi from
erf by Abramowitz & Stegun 7.1.26, |error| <= 1.5e-7) and divide by
den = max(sum gate, 1) (v401:340).

Tolerances: out within 2e-2 relative (Frobenius) of the bf16 restatement; the
gate sum within 2e-3 relative (the erf approximation and fp32 summation
order); den likewise; the passing set (z > 0, i.e. s > tau) identical outside
a tie band of one bf16 score ulp plus the tau slack, with the count inside
the band bounded (tests/parity.py); n_active equal to the mask's popcount.
"""

from __future__ import annotations

import pytest
import torch

from oracle import srw_ref
from tests.parity import REL_BF16, assert_pass_set, bf16_ulp, rel_fro, row_rel_max, unpack_mask

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


def _inputs(pkg, T, D, dr, N, h_is_x, seed, tau):
    shape = pkg.inputs.PoolShape(T=T, D=D, N=N, dr=dr, routes=1, h_is_x=h_is_x)
    inp = pkg.inputs.make_pool_inputs(shape, seed=seed)
    inp["tau_offset"].fill_(tau)
    return inp


def _gpu(pkg, dev, inp, **kw):
    x = inp["x"].to(BF).to(dev)
    h = x if "h" not in inp else inp["h"].to(BF).to(dev)
    res = pkg.srw_forward(x, h, inp["emb"].to(BF).to(dev), inp["tau_offset"].to(dev),
                          inp["read"].to(BF).to(dev), inp["write"].to(BF).to(dev), gate="gelu_v401", **kw)
    torch.cuda.synchronize()
    return {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in res.items()}


def _check_common(got, out_ref, z, s_std, tau, gate_sum_ref, den_ref, T, N, D):
    out = got["out"][:, 0].float()
    err = rel_fro(out, out_ref.reshape(T, D))
    print(f"  out rel err {err:.3e}, worst row {row_rel_max(out, out_ref.reshape(T, D)):.3e}", flush=True)
    assert err <= REL_BF16
    assert row_rel_max(out, out_ref.reshape(T, D)) <= 5e-2
    assert torch.allclose(got["gate_sum"][:, 0], gate_sum_ref.reshape(T), rtol=2e-3, atol=1e-5)
    assert torch.allclose(got["den"][:, 0], den_ref.reshape(T), rtol=2e-3, atol=1e-5)
    # pass <=> z > 0 <=> s - tau > 0; the band: a bf16 score ulp + tau slack
    raw = (z * s_std).reshape(T, N)
    delta = bf16_ulp(raw + tau.reshape(T, 1)) + 1e-4 * s_std.reshape(T, 1)
    mask = unpack_mask(got["pass_mask"][:, 0], N)
    assert_pass_set(mask, raw, delta)
    assert torch.equal(got["n_active"][:, 0].long(), mask.sum(dim=1))


CASES = [
    # T, D, dr, N, h_is_x, max_chunk, tau_offset, seed, path
    (256, 384, 384, 2600, True, 1300, 0.3, 1, "mfma_bf16"),       # h aliases x, chunk edge in a tile
    (200, 384, 128, 1580, False, 12500, 0.8, 2, "mfma_bf16"),     # router h, ragged T and N
    (77, 128, 64, 777, False, 300, 0.0, 3, "mfma_decode_bf16"),  # three chunks, decode kernel
    (64, 384, 128, 25200, False, 12600, 1.2, 4, "mfma_decode_bf16"),  # the Know pool, decode batch
    (130, 128, 128, 70, True, 2048, 0.5, 5, "mfma_bf16"),         # one partial tile
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "T{}D{}dr{}N{}{}c{}".format(
    c[0], c[1], c[2], c[3], "x" if c[4] else "", c[5]))
def test_gelu_v401_mfma_matches_fused_oracle(pkg, dev, case):
    T, D, dr, N, hx, max_chunk, tau, seed, path = case
    print(f"[gpu] gelu v401 mfma {case}", flush=True)
    inp = _inputs(pkg, T, D, dr, N, hx, seed, tau)
    _, cs = srw_ref.chunk_plan(N, max_chunk)
    got = _gpu(pkg, dev, inp, chunk_size=cs, stats="onepass", want_mask=True)
    assert got["path"] == path
    x = inp["x"][None]
    h = x if "h" not in inp else inp["h"][:, 0][None]
    ref, tr = srw_ref.fused_gate_srw_gelu_v401(x, h, inp["emb"], inp["tau_offset"][None], inp["read"],
                                               inp["write"], max_chunk_size=max_chunk, return_trace=True)
    _check_common(got, ref[0], tr["z"], tr["s_std"], tr["tau"], tr["gate_sum"], tr["den"], T, N, D)


def test_gelu_v401_srw_inference_bf16_on_matrix_cores(pkg, dev):
    """srw_inference(gate="gelu_v401") in bf16 -- centred statistics, one
    chunk, s - tau in bf16 (v401:1443-1463) -- runs on the matrix cores."""
    T, D, dr, N = 96, 128, 128, 1500
    print(f"[gpu] gelu v401 srw_inference bf16 T{T} D{D} dr{dr} N{N}", flush=True)
    inp = _inputs(pkg, T, D, dr, N, False, 31, 0.6)
    got = _gpu(pkg, dev, inp, stats="centered", want_mask=True)
    assert got["path"].startswith("mfma")
    h = inp["h"][:, 0]
    out_ref, tr = srw_ref.srw_inference_gelu_v401(inp["x"].to(BF), h.to(BF), inp["emb"].to(BF),
                                                  inp["tau_offset"], inp["read"].to(BF), inp["write"].to(BF),
                                                  return_trace=True)
    gs = tr["gate"].sum(dim=-1)
    _check_common(got, out_ref, tr["z"], tr["s_std"], tr["tau"], gs, tr["den"], T, N, D)


def test_gelu_v401_den_floor_and_no_pass(pkg, dev):
    """tau far above every score: no unit passes, every gate is 0, den = 1
    and out = 0 (v401:340-342)."""
    T, D, dr, N = 48, 128, 128, 640
    print("[gpu] gelu v401 no unit passes", flush=True)
    inp = _inputs(pkg, T, D, dr, N, False, 41, 50.0)
    got = _gpu(pkg, dev, inp, stats="onepass", want_mask=True)
    assert got["path"].startswith("mfma")
    assert bool((got["gate_sum"][:, 0] == 0).all()) and bool((got["den"][:, 0] == 1).all())
    assert bool((got["out"].float() == 0).all())
    assert int(got["n_active"].sum()) == 0


# ---------------------------------------------------------------- v4.0.1 diagnostics
#
# SRW_FLAG_DIAG with the GELU gate (the training forward of v401:230-367, whose
# fused function always returns its diagnostics) on the matrix cores
# (srw_main_ws_kernel<..., DG, GL>) and on the generic kernels, against the
# oracle's trace.  Counts are thresholds on z (phi > 0.95 or < 0.05 <=> |z| >
# Phi^-1(0.95); gate > 0.5 <=> z > z* with z* Phi(z*) = 0.5; the z bands), so
# an element may fall on the other side of an edge only when its z lies
# within the z-shift of one bf16 score ulp plus the tau / s_std slack: the
# count difference is bounded by the number of such elements (+ 2).

V401_DIAG_CASES = [
    # T, D, dr, N, h_is_x, max_chunk, seed
    (256, 384, 384, 6000, True, 2500, 61),    # h aliases x, two reference chunks
    (200, 384, 128, 1580, False, 12500, 62),  # the model's router width, ragged T
    (130, 128, 64, 1000, False, 300, 63),     # four chunks, chunk edges inside tiles
]


def _z_star():
    """z* with z* Phi(z*) = 0.5 (gate > 0.5 <=> z > z*), by bisection in float64."""
    lo, hi = 0.0, 3.0
    for _ in range(80):
        mid = 0.5 * (lo + hi)
        v = mid * 0.5 * (1.0 + torch.erf(torch.tensor(mid / 2 ** 0.5, dtype=torch.float64)))
        lo, hi = (mid, hi) if float(v) < 0.5 else (lo, mid)
    return 0.5 * (lo + hi)


def _check_v401_diag(got, tr, sc, T, N, label):
    """token_diag [T,1,14] / unit_diag [N,2] of one call against the oracle
    trace (z, gate, tau, s_std) and the oracle's bf16 scores sc [T, N]."""
    td = got["token_diag"][:, 0].double()
    z = tr["z"].reshape(T, N).double()
    gate = tr["gate"].reshape(T, N).double()
    s_std = tr["s_std"].reshape(T).double()
    names = ["s_mean", "s_std", "tau", "sum_s3", "sum_s4", "gate_max", "int_sum", "n_strong",
             "n_boundary", "n_band075", "n_band030", "g_log_g", "int_max", "n_int_cap"]
    col = {n: i for i, n in enumerate(names)}
    assert torch.allclose(td[:, col["s_mean"]], tr["s_mean"].reshape(T).double(), rtol=1e-4, atol=1e-5)
    assert torch.allclose(td[:, col["s_std"]], s_std, rtol=1e-4, atol=1e-5)
    assert torch.allclose(td[:, col["tau"]], tr["tau"].reshape(T).double(), rtol=1e-4, atol=1e-5)
    sc = sc.double()
    sens = (3 * sc.abs() ** 2 * bf16_ulp(sc)).sum(dim=-1)
    d3 = (td[:, col["sum_s3"]] - (sc ** 3).sum(-1)).abs()
    assert (d3 <= 0.02 * sens + 1e-5 * (sc.abs() ** 3).sum(-1)).all(), label
    assert torch.allclose(td[:, col["gate_max"]], gate.amax(-1), rtol=2e-3, atol=1e-6), label
    assert torch.allclose(td[:, col["int_sum"]], z.clamp_min(0).sum(-1), rtol=2e-3, atol=1e-4), label
    mag = (gate * torch.log(gate + 1e-8)).abs().sum(-1)
    d = (td[:, col["g_log_g"]] - (gate * torch.log(gate + 1e-8)).sum(-1)).abs()
    assert (d <= 1e-3 + 2e-3 * mag).all(), label
    assert bool((td[:, col["int_max"]] == 0).all()) and bool((td[:, col["n_int_cap"]] == 0).all())
    # counts, with the tie band in z
    dz = (bf16_ulp(sc) + 1e-4 * s_std[:, None]) / s_std[:, None] + 1e-5
    zs, z95 = _z_star(), 1.6448536269514722
    preds = {
        "n_strong": (z > zs, (zs,)),
        "n_boundary": (z.abs() > z95, (z95, -z95)),
        "n_band075": ((z > 0) & (z < 0.75), (0.0, 0.75)),
        "n_band030": ((z > 0) & (z < 0.30), (0.0, 0.30)),
    }
    for n, (pred, edges) in preds.items():
        band = sum(((z - c).abs() <= dz).sum(-1) for c in edges)
        diff = (td[:, col[n]] - pred.sum(-1)).abs()
        print(f"  {label} {n}: max |diff| {float(diff.max())}, max band {int(band.max())}", flush=True)
        assert (diff <= band + 2).all(), (label, n)
    # per-unit score sums: a score may round to the neighbouring bf16 value
    # (the two sides sum its products in another order, ~1 in 10^3): bound the
    # difference by four of the unit's largest score ulps plus 2% of its
    # summed ulps (a missing or repeated 32-row block moves a sum by ~32 |s|)
    ud = got["unit_diag"].double()
    d = (ud[:, 0] - sc.sum(0)).abs()
    ulp = bf16_ulp(sc)
    bound = 4 * ulp.amax(0) + 0.02 * ulp.sum(0) + 1e-5 * sc.abs().sum(0)
    print(f"  {label} unit score_sum: max |diff| {float(d.max()):.3e}, max diff/bound "
          f"{float((d / bound).max()):.3f}", flush=True)
    assert (d <= bound).all(), label
    assert torch.allclose(ud[:, 1], gate.amax(0), rtol=2e-3, atol=1e-5), label


@pytest.mark.parametrize("case", V401_DIAG_CASES, ids=lambda c: "T{}D{}dr{}N{}{}c{}".format(
    c[0], c[1], c[2], c[3], "x" if c[4] else "", c[5]))
def test_gelu_v401_diagnostics_match_oracle(pkg, dev, case):
    T, D, dr, N, hx, max_chunk, seed = case
    print(f"[gpu] gelu v401 diagnostics {case}", flush=True)
    inp = _inputs(pkg, T, D, dr, N, hx, seed, 0.0)
    inp["tau_offset"].uniform_(-0.6, 1.2, generator=torch.Generator().manual_seed(seed))
    _, cs = srw_ref.chunk_plan(N, max_chunk)
    fast = _gpu(pkg, dev, inp, chunk_size=cs, stats="onepass", want_mask=True, diag=True)
    plain = _gpu(pkg, dev, inp, chunk_size=cs, stats="onepass", want_mask=True)
    slow = _gpu(pkg, dev, inp, chunk_size=cs, stats="onepass", want_mask=True, diag=True, emulate=True)
    assert fast["path"] == "mfma_bf16" and plain["path"] == "mfma_bf16" and slow["path"] == "generic"
    # diagnostics leave the forward's results unchanged, bit for bit
    for k in ("out", "gate_sum", "den", "n_active", "pass_mask"):
        assert torch.equal(fast[k], plain[k]), k
    x = inp["x"][None]
    h = x if hx else inp["h"][:, 0][None]
    ref, tr = srw_ref.fused_gate_srw_gelu_v401(x, h, inp["emb"], inp["tau_offset"][None], inp["read"],
                                               inp["write"], max_chunk_size=max_chunk, return_trace=True)
    _check_common(fast, ref[0], tr["z"], tr["s_std"], tr["tau"], tr["gate_sum"], tr["den"], T, N, D)
    hh = (inp["x"] if hx else inp["h"][:, 0]).to(BF).float()
    sc = (hh @ inp["emb"].to(BF).float().T).to(BF).float()       # bf16 scores (v401:251)
    _check_v401_diag(fast, tr, sc, T, N, "mfma")
    _check_v401_diag(slow, tr, sc, T, N, "generic")


@pytest.mark.parametrize("hx", [False, True], ids=["router_h", "h_is_x"])
def test_dropin_v401_16_tuple(pkg, dev, hx):
    """make_sharded_srw_v401 (v401:194-369) against the oracle's 16-tuple."""
    B, S, D, N = 2, 40, 128, 1200
    dr = D if hx else 64
    print(f"[gpu] drop-in v401 16-tuple B{B} S{S} D{D} dr{dr} N{N} hx={hx}", flush=True)
    inp = _inputs(pkg, B * S, D, dr, N, hx, 71, 0.0)
    inp["tau_offset"].uniform_(-0.5, 1.0, generator=torch.Generator().manual_seed(71))
    x = inp["x"].reshape(B, S, D)
    h = x if hx else inp["h"].reshape(B, S, dr)
    tau = inp["tau_offset"].reshape(B, S, 1)
    fn = pkg.make_sharded_srw_v401(None, max_chunk_size=500)
    xd = x.to(dev)
    got = fn(xd, xd if hx else h.to(dev), inp["emb"].to(dev), tau.to(dev), inp["read"].to(dev),
             inp["write"].to(dev))
    torch.cuda.synchronize()
    ref = srw_ref.fused_gate_srw_gelu_v401(x, h, inp["emb"], tau, inp["read"], inp["write"],
                                           max_chunk_size=500)
    assert len(got) == 16
    assert rel_fro(got[0].cpu(), ref[0]) <= REL_BF16
    for i, name in enumerate(srw_ref.FUSED_V401_OUTPUT_NAMES[1:], start=1):
        g, r = got[i].detach().cpu().float(), ref[i].float()
        assert g.shape == r.shape, name
        assert torch.allclose(g, r, rtol=2e-2, atol=2e-3), (name, g, r)


def test_dropin_v401_paired_16_tuple(pkg, dev):
    """make_sharded_srw_paired_v401 (v401:372-554) against the oracle's paired
    16-tuple; the call runs on the matrix cores (two routes, GELU gate,
    diagnostics)."""
    B, S, D, dr, N = 2, 40, 128, 64, 1200
    print(f"[gpu] drop-in v401 paired 16-tuple B{B} S{S} D{D} dr{dr} N{N}", flush=True)
    shape = pkg.inputs.PoolShape(T=B * S, D=D, N=N, dr=dr, routes=2, h_is_x=False)
    inp = pkg.inputs.make_pool_inputs(shape, seed=81)
    inp["tau_offset"].uniform_(-0.5, 1.0, generator=torch.Generator().manual_seed(81))
    x = inp["x"].reshape(B, S, D)
    h = inp["h"].reshape(B, S, 2, dr)
    tau = inp["tau_offset"].reshape(B, S, 2, 1)
    fn = pkg.make_sharded_srw_paired_v401(None, max_chunk_size=500)
    got = fn(x.to(dev), h.to(dev), inp["emb"].to(dev), tau.to(dev), inp["read"].to(dev), inp["write"].to(dev))
    torch.cuda.synchronize()
    ref = srw_ref.fused_gate_srw_gelu_v401_paired(x, h, inp["emb"], tau, inp["read"], inp["write"],
                                                  max_chunk_size=500)
    assert len(got) == 16 and got[0].shape == (B, S, 2, D)
    assert rel_fro(got[0].cpu(), ref[0]) <= REL_BF16
    for i, name in enumerate(srw_ref.FUSED_V401_OUTPUT_NAMES[1:], start=1):
        g, r = got[i].detach().cpu().float(), ref[i].float()
        assert g.shape == r.shape, name
        assert torch.allclose(g, r, rtol=2e-2, atol=2e-3), (name, g, r)
    # the same call through srw_forward names its kernel family
    _, cs = srw_ref.chunk_plan(N, 500)
    res = pkg.srw_forward(inp["x"].to(BF).to(dev), inp["h"].to(BF).to(dev), inp["emb"].to(BF).to(dev),
                          inp["tau_offset"].to(dev), inp["read"].to(BF).to(dev), inp["write"].to(BF).to(dev),
                          gate="gelu_v401", stats="onepass", chunk_size=cs, diag=True, want_mask=False)
    assert res["path"] == "mfma_bf16"
