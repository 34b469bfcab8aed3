"""GPU parity of srw_backward (the VJP of fused_gate_srw, through the C ABI)
against the oracle's hand-written VJP (oracle/srw_vjp.py) with the
reference's bf16 rounding points, on the same seeded inputs.

Bar: every gradient within 2e-2 relative (Frobenius) of the oracle's, and
d tau_offset within 2e-2 relative per token row set.  The two sides differ
by fp32 accumulation order inside the bf16 dots (a score or a product can
round to the neighbouring bf16 value) and by where a cotangent is rounded
when two paths meet (documented in the oracle).
"""

from __future__ import annotations

import pytest
import torch

from oracle import srw_vjp
from tests.parity import rel_fro

pytestmark = pytest.mark.gpu

BF = torch.bfloat16

CASES = [
    # T, D, dr, N, h_is_x, seed, tau
    (256, 384, 384, 2600, True, 1, -0.5),     # Know-pool form, ragged N
    (200, 384, 128, 1580, False, 2, -0.5),    # router h, ragged T and N
    (130, 128, 64, 1000, False, 3, 0.5),      # fewer passing units
    (64, 1024, 1024, 700, True, 4, -0.5),     # configs[4] widths
    (40, 128, 128, 300, True, 5, 2.5),        # dead units (score_lb / dead penalty terms)
]


def _inputs(pkg, T, D, dr, N, hx, seed, tau):
    shape = pkg.inputs.PoolShape(T=T, D=D, N=N, dr=dr, routes=1, h_is_x=hx)
    inp = pkg.inputs.make_pool_inputs(shape, seed=seed)
    g = torch.Generator().manual_seed(seed + 7)
    inp["tau_offset"] = tau + 0.2 * torch.randn(T, 1, generator=g)
    return inp


@pytest.mark.parametrize("case", CASES, ids=lambda c: "T{}D{}dr{}N{}{}".format(
    c[0], c[1], c[2], c[3], "x" if c[4] else ""))
def test_backward_matches_oracle_vjp(pkg, dev, case):
    T, D, dr, N, hx, seed, tau = case
    print(f"[gpu] backward {case}", flush=True)
    inp = _inputs(pkg, T, D, dr, N, hx, seed, tau)
    xb = inp["x"].to(BF)
    hb = xb if hx else inp["h"][:, 0].to(BF)
    eb, rb, wb = (inp[k].to(BF) for k in ("emb", "read", "write"))
    g = torch.Generator().manual_seed(seed + 99)
    d_out = torch.randn(T, D, generator=g)
    d_lb, d_pen = 0.37, -0.81
    ref = srw_vjp.fused_gate_srw_vjp(xb.float(), hb.float(), eb.float(), inp["tau_offset"], rb.float(),
                                     wb.float(), d_out, d_lb, d_pen, max_chunk_size=max(N, 1))
    x = xb.to(dev)
    h = x if hx else hb[:, None].contiguous().to(dev)
    args = (x, h, eb.to(dev), inp["tau_offset"].to(dev), rb.to(dev), wb.to(dev))
    fwd = pkg.srw_forward(*args, want_mask=False)
    got = pkg.srw_backward(*args, fwd["out"], d_out[:, None].to(dev), d_lb, d_pen)
    torch.cuda.synchronize()
    assert got["path"] == "tiled_bwd_bf16"
    pairs = dict(dx=got["dx"], dh=got["dh"][:, 0], demb=got["demb"], dtau_offset=got["dtau_offset"],
                 dread=got["dread"], dwrite=got["dwrite"])
    for k, v in pairs.items():
        err = rel_fro(v.cpu(), ref[k].float())
        print(f"  {k}: rel err {err:.3e}", flush=True)
        assert torch.isfinite(v).all(), k
        assert err <= 2e-2, (k, err)


@pytest.mark.parametrize("case", [CASES[0], CASES[1], CASES[4]], ids=lambda c: "T{}D{}dr{}N{}{}".format(
    c[0], c[1], c[2], c[3], "x" if c[4] else ""))
def test_backward_with_forward_residuals(pkg, dev, case):
    """With the forward's den and unit diagnostics handed over (the drop-in's
    training path) the backward skips its own pass over the scores for them:
    every gradient still within the oracle bar, and within 1e-2 of the
    backward that recomputes them (the two differ by the forward's summation
    order of den and the unit score sums)."""
    T, D, dr, N, hx, seed, tau = case
    print(f"[gpu] backward with residuals {case}", flush=True)
    inp = _inputs(pkg, T, D, dr, N, hx, seed, tau)
    xb = inp["x"].to(BF)
    hb = xb if hx else inp["h"][:, 0].to(BF)
    eb, rb, wb = (inp[k].to(BF) for k in ("emb", "read", "write"))
    g = torch.Generator().manual_seed(seed + 99)
    d_out = torch.randn(T, D, generator=g)
    d_lb, d_pen = 0.37, -0.81
    ref = srw_vjp.fused_gate_srw_vjp(xb.float(), hb.float(), eb.float(), inp["tau_offset"], rb.float(),
                                     wb.float(), d_out, d_lb, d_pen, max_chunk_size=max(N, 1))
    x = xb.to(dev)
    h = x if hx else hb[:, None].contiguous().to(dev)
    args = (x, h, eb.to(dev), inp["tau_offset"].to(dev), rb.to(dev), wb.to(dev))
    fwd = pkg.srw_forward(*args, want_mask=False, diag=True)
    got = pkg.srw_backward(*args, fwd["out"], d_out[:, None].to(dev), d_lb, d_pen,
                           den=fwd["den"], unit_diag=fwd["unit_diag"])
    plain = pkg.srw_backward(*args, fwd["out"], d_out[:, None].to(dev), d_lb, d_pen)
    torch.cuda.synchronize()
    pairs = dict(dx=(got["dx"], plain["dx"]), dh=(got["dh"][:, 0], plain["dh"][:, 0]),
                 demb=(got["demb"], plain["demb"]), dtau_offset=(got["dtau_offset"], plain["dtau_offset"]),
                 dread=(got["dread"], plain["dread"]), dwrite=(got["dwrite"], plain["dwrite"]))
    for k, (v, w) in pairs.items():
        err = rel_fro(v.cpu(), ref[k].float())
        same = rel_fro(v.cpu(), w.cpu())
        print(f"  {k}: rel err {err:.3e}, against the recomputing backward {same:.3e}", flush=True)
        assert torch.isfinite(v).all(), k
        assert err <= 2e-2, (k, err)
        assert same <= 1e-2, (k, same)


def test_backward_residuals_both_or_neither(pkg, dev):
    """den without unit_diag (or the reverse) is refused."""
    T, D, N = 32, 128, 300
    x = torch.randn(T, D, device=dev).to(BF)
    emb = torch.randn(N, D, device=dev).to(BF)
    rw = torch.randn(N, D, device=dev).to(BF)
    tau = torch.full((T, 1), -0.5, device=dev)
    out = torch.zeros(T, 1, D, dtype=BF, device=dev)
    d_out = torch.zeros(T, 1, D, device=dev)
    with pytest.raises(ValueError):
        pkg.srw_backward(x, x, emb, tau, rw, rw, out, d_out, 0.0, 0.0, den=torch.ones(T, 1, device=dev))


def test_backward_linear_in_cotangents(pkg, dev):
    """The VJP is linear in (d_out, d_lb, d_pen): grad(a + b) = grad(a) + grad(b)
    up to the bf16 rounding of each contraction."""
    T, D, dr, N = 128, 384, 384, 1500
    print(f"[gpu] backward linearity T{T} N{N}", flush=True)
    inp = _inputs(pkg, T, D, dr, N, True, 11, -0.5)
    x = inp["x"].to(BF).to(dev)
    args = (x, x, inp["emb"].to(BF).to(dev), inp["tau_offset"].to(dev), inp["read"].to(BF).to(dev),
            inp["write"].to(BF).to(dev))
    out = pkg.srw_forward(*args, want_mask=False)["out"]
    g = torch.Generator().manual_seed(5)
    da = torch.randn(T, 1, D, generator=g).to(dev)
    db = torch.randn(T, 1, D, generator=g).to(dev)
    ga = pkg.srw_backward(*args, out, da, 0.5, 0.0)
    gb = pkg.srw_backward(*args, out, db, 0.0, -1.0)
    gs = pkg.srw_backward(*args, out, da + db, 0.5, -1.0)
    torch.cuda.synchronize()
    for k in ("dx", "dh", "demb", "dtau_offset", "dread", "dwrite"):
        err = rel_fro((ga[k] + gb[k]).cpu(), gs[k].cpu())
        assert err <= 2e-2, (k, err)


@pytest.mark.parametrize("case", [(96, 384, 128, 1580, 21), (70, 128, 64, 777, 22)],
                         ids=lambda c: "T{}D{}dr{}N{}".format(*c[:4]))
def test_backward_paired_matches_oracle(pkg, dev, case):
    """Paired QK routes (fused_gate_srw_paired, v41:640-909): rows are (token,
    route) pairs sharing one x.R^T; the oracle is the single-route VJP on
    those 2T rows with x repeated per route, dx summed over a token's routes."""
    T, D, dr, N, seed = case
    print(f"[gpu] backward paired {case}", flush=True)
    shape = pkg.inputs.PoolShape(T=T, D=D, N=N, dr=dr, routes=2)
    inp = pkg.inputs.make_pool_inputs(shape, seed=seed)
    g = torch.Generator().manual_seed(seed + 7)
    tau = -0.5 + 0.2 * torch.randn(T, 2, generator=g)
    xb = inp["x"].to(BF)
    hb = inp["h"].to(BF)
    eb, rb, wb = (inp[k].to(BF) for k in ("emb", "read", "write"))
    d_out = torch.randn(T, 2, D, generator=g)
    d_lb, d_pen = 0.4, -0.6
    ref = srw_vjp.fused_gate_srw_vjp(xb.float().repeat_interleave(2, dim=0), hb.float().reshape(2 * T, dr),
                                     eb.float(), tau.reshape(2 * T, 1), rb.float(), wb.float(),
                                     d_out.reshape(2 * T, D), d_lb, d_pen, max_chunk_size=N)
    args = (xb.to(dev), hb.to(dev), eb.to(dev), tau.to(dev), rb.to(dev), wb.to(dev))
    fwd = pkg.srw_forward(*args, want_mask=False)
    got = pkg.srw_backward(*args, fwd["out"], d_out.to(dev), d_lb, d_pen)
    torch.cuda.synchronize()
    want = dict(dx=ref["dx"].reshape(T, 2, D).sum(dim=1), dh=ref["dh"].reshape(T, 2, dr), demb=ref["demb"],
                dtau_offset=ref["dtau_offset"].reshape(T, 2), dread=ref["dread"], dwrite=ref["dwrite"])
    for k, v in want.items():
        err = rel_fro(got[k].cpu(), v.float())
        print(f"  {k}: rel err {err:.3e}", flush=True)
        assert err <= 2e-2, (k, err)


def test_backward_scale_and_dscale(pkg, dev):
    """A scale folded into the call (the caller's *_scale multiply, v41:1044-1053,
    1175): at scale 2 (a power of two, so every rounding commutes with it) the
    gradients equal those at scale 1 with the cotangent doubled, bit for bit;
    dscale equals <d_out, out at scale 1> from the oracle's forward."""
    T, D, dr, N, seed = 96, 384, 128, 1580, 31
    print(f"[gpu] backward scale T{T} N{N}", flush=True)
    inp = _inputs(pkg, T, D, dr, N, False, seed, -0.5)
    xb = inp["x"].to(BF)
    hb = inp["h"][:, 0].to(BF)
    eb, rb, wb = (inp[k].to(BF) for k in ("emb", "read", "write"))
    g = torch.Generator().manual_seed(seed)
    d_out = torch.randn(T, D, generator=g)
    args = (xb.to(dev), hb[:, None].contiguous().to(dev), eb.to(dev), inp["tau_offset"].to(dev), rb.to(dev),
            wb.to(dev))
    out1 = pkg.srw_forward(*args, want_mask=False)["out"]
    out2 = pkg.srw_forward(*args, want_mask=False, scale=2.0)["out"]
    g1 = pkg.srw_backward(*args, out1, (2.0 * d_out)[:, None].to(dev), 0.3, -0.7)
    g2 = pkg.srw_backward(*args, out2, d_out[:, None].to(dev), 0.3, -0.7, scale=2.0)
    torch.cuda.synchronize()
    assert torch.equal(out2.float(), 2.0 * out1.float())
    for k in ("dx", "dh", "demb", "dtau_offset", "dread", "dwrite"):
        assert torch.equal(g1[k], g2[k]), k
    ref = srw_vjp.fused_gate_srw_vjp(xb.float(), hb.float(), eb.float(), inp["tau_offset"], rb.float(),
                                     wb.float(), d_out, 0.3, -0.7, max_chunk_size=N)
    want = float((d_out.double() * ref["out"].double()).sum())
    got = float(g2["dscale"])
    print(f"  dscale {got:.6f} oracle {want:.6f}", flush=True)
    assert abs(got - want) <= 1e-2 * abs(want) + 1e-3


def test_backward_empty_tokens(pkg, dev):
    """T = 0: nothing flows into the pool, whose gradients are zero."""
    D, N = 128, 300
    z = torch.empty(0, D, dtype=BF, device=dev)
    emb = torch.randn(N, D, device=dev).to(BF)
    rw = torch.randn(N, D, device=dev).to(BF)
    got = pkg.srw_backward(z, z, emb, torch.empty(0, 1, device=dev), rw, rw,
                           torch.empty(0, 1, D, dtype=BF, device=dev), torch.empty(0, 1, D, device=dev), 0.5, 0.5)
    torch.cuda.synchronize()
    for k in ("demb", "dread", "dwrite", "dscale"):
        assert torch.count_nonzero(got[k]) == 0, k
    assert got["dx"].shape == (0, D) and got["dtau_offset"].shape == (0, 1)
