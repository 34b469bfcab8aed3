"""GPU parity of srw_backward with the v4.0.1 GELU gate (the VJP of the
legacy fused_gate_srw, models/legacy/dawn_spatial_v401_exp.py:229-554,
through the C ABI) against torch autograd through the oracle's bf16
restatement of that forward (``srw_ref.fused_gate_srw_gelu_v401``, pinned on
the CPU in tests/test_oracle_pins.py).  The oracle's bf16 roundings are
casts, whose transposes round the cotangents to bf16 where the reference's
JAX autodiff does; autograd through a pinned forward is that forward's
gradient.  Loss: <d_out, out> + d_lb * score_lb (out and lb_loss, the
outputs the v4.0.1 callers' losses use, v401:909, 978).

Bar: every gradient within 2e-2 relative (Frobenius) of the oracle's, as for
the v4.1 backward (tests/test_gpu_backward.py).
"""

from __future__ import annotations

import pytest
import torch

from oracle import srw_ref
from tests.parity import rel_fro

pytestmark = pytest.mark.gpu

BF = torch.bfloat16

CASES = [
    # T, D, dr, N, h_is_x, routes, seed, max_chunk
    (256, 384, 384, 2600, True, 1, 1, 1300),     # Know-pool form, two reference chunks
    (200, 384, 128, 1580, False, 1, 2, 12500),   # router h, ragged T and N
    (130, 128, 64, 1000, False, 1, 3, 300),      # four chunks
    (96, 384, 128, 1580, False, 2, 4, 12500),    # paired routes
    (64, 1024, 1024, 700, True, 1, 5, 12500),    # configs[4] widths: the products on the 256 x 256 tiles
]


def _oracle_grads(x, h, e, tau, r, w, d_out, d_lb, hx, routes, max_chunk):
    """Autograd of <d_out, out> + d_lb score_lb through the bf16 oracle."""
    T, D = x.shape
    leaves = [t.clone().requires_grad_(True) for t in (x, e, tau, r, w)]
    xl, el, taul, rl, wl = leaves
    hl = None if hx else h.clone().requires_grad_(True)
    if routes == 1:
        res = srw_ref.fused_gate_srw_gelu_v401(xl[None], (xl if hx else hl)[None], el, taul[None], rl, wl,
                                               max_chunk_size=max_chunk)
        loss = (res[0][0] * d_out[:, 0]).sum()
    else:
        res = srw_ref.fused_gate_srw_gelu_v401_paired(xl[None], hl[None], el, taul.reshape(1, T, 2, 1), rl, wl,
                                                      max_chunk_size=max_chunk)
        loss = (res[0][0] * d_out).sum()
    loss = loss + d_lb * res[3]
    loss.backward()
    out = dict(dx=xl.grad, demb=el.grad, dtau_offset=taul.grad.reshape(T, routes), dread=rl.grad,
               dwrite=wl.grad)
    if not hx:
        out["dh"] = hl.grad
    return out


@pytest.mark.parametrize("residuals", [False, True], ids=["recompute", "residuals"])
@pytest.mark.parametrize("case", CASES, ids=lambda c: "T{}D{}dr{}N{}{}R{}".format(
    c[0], c[1], c[2], c[3], "x" if c[4] else "", c[5]))
def test_v401_backward_matches_oracle_autograd(pkg, dev, case, residuals):
    T, D, dr, N, hx, R, seed, max_chunk = case
    print(f"[gpu] v401 backward {case} residuals={residuals}", flush=True)
    shape = pkg.inputs.PoolShape(T=T, D=D, N=N, dr=dr, routes=R, h_is_x=hx)
    inp = pkg.inputs.make_pool_inputs(shape, seed=seed)
    g = torch.Generator().manual_seed(seed + 7)
    tau = (0.3 + 0.3 * torch.randn(T, R, generator=g))
    # the R and W rows away from unit norm, so that the forward normalisation matters
    scale_r = 0.5 + 2.0 * torch.rand(N, 1, generator=g)
    scale_w = 0.5 + 2.0 * torch.rand(N, 1, generator=g)
    xb = inp["x"].to(BF)
    hb = xb if hx else inp["h"].to(BF)                      # [T, R, dr]
    eb = inp["emb"].to(BF)
    rb = (inp["read"] * scale_r).to(BF)
    wb = (inp["write"] * scale_w).to(BF)
    d_out = torch.randn(T, R, D, generator=g)
    d_lb = 0.37
    _, cs = srw_ref.chunk_plan(N, max_chunk)
    x = xb.to(dev)
    h = x if hx else hb.contiguous().to(dev)
    args = (x, h, eb.to(dev), tau.to(dev), rb.to(dev), wb.to(dev))
    fwd = pkg.srw_forward(*args, gate="gelu_v401", stats="onepass", chunk_size=cs, want_mask=False,
                          diag=residuals)
    kw = dict(den=fwd["den"], unit_diag=fwd["unit_diag"]) if residuals else {}
    got = pkg.srw_backward(*args, fwd["out"], d_out.to(dev), d_lb, 0.0, gate="gelu_v401", **kw)
    torch.cuda.synchronize()
    assert got["path"] == "tiled_bwd_bf16"
    h_ref = None if hx else (hb[:, 0] if R == 1 else hb).float()
    ref = _oracle_grads(xb.float(), h_ref, eb.float(), tau, rb.float(), wb.float(), d_out, d_lb, hx, R, max_chunk)
    pairs = dict(dx=got["dx"] + (got["dh"][:, 0] if hx else 0), demb=got["demb"],
                 dtau_offset=got["dtau_offset"], dread=got["dread"], dwrite=got["dwrite"])
    if not hx:
        pairs["dh"] = got["dh"][:, 0] if R == 1 else got["dh"]
    for k, v in pairs.items():
        err = rel_fro(v.cpu(), ref[k].float())
        print(f"  {k}: rel err {err:.3e}", flush=True)
        assert torch.isfinite(v).all(), k
        assert err <= 2e-2, (k, err)


def test_v401_backward_refuses_dead_penalty(pkg, dev):
    """The v4.0.1 function has no dead_penalty: a cotangent for it is refused
    before any launch."""
    T, D, dr, N = 32, 128, 64, 200
    shape = pkg.inputs.PoolShape(T=T, D=D, N=N, dr=dr, routes=1, h_is_x=False)
    inp = pkg.inputs.make_pool_inputs(shape, seed=9)
    args = (inp["x"].to(BF).to(dev), inp["h"].to(BF).to(dev), inp["emb"].to(BF).to(dev),
            inp["tau_offset"].to(dev), inp["read"].to(BF).to(dev), inp["write"].to(BF).to(dev))
    fwd = pkg.srw_forward(*args, gate="gelu_v401", stats="onepass", want_mask=False)
    with pytest.raises(pkg.SrwError):
        pkg.srw_backward(*args, fwd["out"], torch.zeros(T, 1, D, device=dev), 0.0, 0.5, gate="gelu_v401")


def test_dropin_v401_autograd(pkg, dev):
    """make_sharded_srw_v401's autograd node: loss = <c, out> + 0.3 score_lb
    backpropagates to the six inputs as autograd through the oracle does."""
    B, S, D, dr, N = 2, 48, 128, 64, 900
    print(f"[gpu] drop-in v401 autograd B{B} S{S} D{D} dr{dr} N{N}", flush=True)
    shape = pkg.inputs.PoolShape(T=B * S, D=D, N=N, dr=dr, routes=1, h_is_x=False)
    inp = pkg.inputs.make_pool_inputs(shape, seed=11)
    g = torch.Generator().manual_seed(12)
    c = torch.randn(B, S, D, generator=g)
    tau = (0.2 + 0.3 * torch.randn(B, S, 1, generator=g))
    host = dict(x=inp["x"].reshape(B, S, D), h=inp["h"].reshape(B, S, dr), emb=inp["emb"], tau=tau,
                read=inp["read"], write=inp["write"])
    host = {k: v.to(BF).float() if k != "tau" else v for k, v in host.items()}
    leaves = {k: v.to(dev).requires_grad_(True) for k, v in host.items()}
    fn = pkg.make_sharded_srw_v401(None, max_chunk_size=450)
    res = fn(leaves["x"], leaves["h"], leaves["emb"], leaves["tau"], leaves["read"], leaves["write"])
    (res[0] * c.to(dev)).sum().add(0.3 * res[3]).backward()
    torch.cuda.synchronize()
    ref_leaves = {k: v.clone().requires_grad_(True) for k, v in host.items()}
    ref = srw_ref.fused_gate_srw_gelu_v401(ref_leaves["x"], ref_leaves["h"], ref_leaves["emb"], ref_leaves["tau"],
                                           ref_leaves["read"], ref_leaves["write"], max_chunk_size=450)
    (ref[0] * c).sum().add(0.3 * ref[3]).backward()
    for k in leaves:
        err = rel_fro(leaves[k].grad.cpu(), ref_leaves[k].grad)
        print(f"  d{k}: rel err {err:.3e}", flush=True)
        assert err <= 2e-2, (k, err)
