"""Pins for the oracle's SRW backward (oracle/srw_vjp.py), CPU only.

The reference trains through fused_gate_srw with JAX autodiff
(models/dawn_spatial_v41_exp.py:415-635, scripts/train_jax.py:726) and ships
no gradient vectors, so the hand-written VJP is pinned by:

* its forward (``fused_terms``) equal to the full forward restatement
  ``srw_ref.fused_gate_srw`` on the three outputs that enter the loss;
* the exact-arithmetic VJP equal to torch autograd of the exact forward in
  fp64 (a dropped term or a wrong sign fails here);
* autograd against central finite differences of the exact forward (fp64),
  along random directions, for every input;
* with the bf16 forward and exact cotangents, the VJP equal to autograd
  through a straight-through rounding (fp64);
* the bf16 cotangent roundings within bf16 tolerance of exact cotangents.
"""

from __future__ import annotations

import pytest
import torch

from oracle import srw_ref, srw_vjp

F64 = torch.float64
NAMES = ("x", "h", "emb", "tau_offset", "read", "write")


def _inputs(T, D, dr, N, seed, tau=-0.5):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, D, generator=g)
    x = x / torch.sqrt((x * x).mean(dim=-1, keepdim=True) + 1e-6)
    h = torch.randn(T, dr, generator=g)
    h = h / torch.sqrt((h * h).mean(dim=-1, keepdim=True) + 1e-6)
    emb = torch.randn(N, dr, generator=g) / dr ** 0.5
    read = torch.randn(N, D, generator=g)
    read = read / read.norm(dim=-1, keepdim=True)
    write = torch.randn(N, D, generator=g)
    write = write / write.norm(dim=-1, keepdim=True)
    tau_off = torch.full((T, 1), tau) + 0.3 * torch.randn(T, 1, generator=g)
    return dict(x=x, h=h, emb=emb, tau_offset=tau_off, read=read, write=write)


def _cot(T, D, seed):
    g = torch.Generator().manual_seed(seed + 1000)
    return torch.randn(T, D, generator=g), 0.7, -1.3


def test_terms_match_full_forward():
    """fused_terms (bf16) reproduces out / score_lb / dead_penalty of the
    22-tuple restatement (v41:630-635 order: index 0, 3, 18)."""
    inp = _inputs(12, 32, 16, 300, seed=1)
    out, lb, pen = srw_vjp.fused_terms(**inp, max_chunk_size=100)
    ref = srw_ref.fused_gate_srw(inp["x"][None], inp["h"][None], inp["emb"], inp["tau_offset"][None],
                                 inp["read"], inp["write"], max_chunk_size=100)
    assert torch.allclose(out, ref[0][0], rtol=0, atol=1e-6)
    assert torch.allclose(lb, ref[3], rtol=1e-5, atol=1e-7)
    assert torch.allclose(pen, ref[18], rtol=1e-5, atol=1e-7)
    # dead units exist in this case (a high tau offset on a tiny token set)
    inp2 = _inputs(4, 32, 16, 300, seed=2, tau=2.5)
    _, _, pen2 = srw_vjp.fused_terms(**inp2, max_chunk_size=300)
    ref2 = srw_ref.fused_gate_srw(inp2["x"][None], inp2["h"][None], inp2["emb"], inp2["tau_offset"][None],
                                  inp2["read"], inp2["write"], max_chunk_size=300)
    assert float(ref2[19]) > 0 and torch.allclose(pen2, ref2[18], rtol=1e-5, atol=1e-7)


def _autograd(inp, d_out, d_lb, d_pen, chunk, rb=srw_vjp.rb_exact):
    leaves = {k: v.to(F64).clone().requires_grad_(True) for k, v in inp.items()}
    out, lb, pen = srw_vjp.fused_terms(**leaves, max_chunk_size=chunk, rb=rb, dtype=F64)
    loss = (out * d_out.to(F64)).sum() + d_lb * lb + d_pen * pen
    grads = torch.autograd.grad(loss, [leaves[k] for k in NAMES])
    return dict(zip(NAMES, grads))


@pytest.mark.parametrize("case", [(8, 24, 16, 120, 40, 3, -0.5), (6, 16, 16, 90, 90, 4, 1.2)])
def test_exact_vjp_equals_autograd(case):
    T, D, dr, N, chunk, seed, tau = case
    inp = _inputs(T, D, dr, N, seed, tau)
    d_out, d_lb, d_pen = _cot(T, D, seed)
    ag = _autograd(inp, d_out, d_lb, d_pen, chunk)
    an = srw_vjp.fused_gate_srw_vjp(**inp, d_out=d_out, d_lb=d_lb, d_pen=d_pen, max_chunk_size=chunk,
                                    rb=srw_vjp.rb_exact, dtype=F64)
    keymap = dict(x="dx", h="dh", emb="demb", tau_offset="dtau_offset", read="dread", write="dwrite")
    for k in NAMES:
        a, b = ag[k], an[keymap[k]]
        assert a.shape == b.shape, k
        err = (a - b).abs().max() / a.abs().max().clamp_min(1e-30)
        assert err < 1e-9, (k, float(err))


def test_autograd_matches_finite_differences():
    """Directional derivatives of the exact forward (fp64) along random
    directions, against the autograd gradient; the steep sigmoid (sharpness
    500) sets the step: margins stay far from the kinks at this size."""
    T, D, dr, N = 6, 16, 12, 80
    inp = {k: v.to(F64) for k, v in _inputs(T, D, dr, N, seed=5).items()}
    d_out, d_lb, d_pen = _cot(T, D, 5)
    ag = _autograd(inp, d_out, d_lb, d_pen, 40)

    def f(vals):
        out, lb, pen = srw_vjp.fused_terms(**vals, max_chunk_size=40, rb=srw_vjp.rb_exact, dtype=F64)
        return float((out * d_out.to(F64)).sum() + d_lb * lb + d_pen * pen)

    g = torch.Generator().manual_seed(77)
    eps = 1e-7
    for k in NAMES:
        for _ in range(3):
            v = torch.randn(inp[k].shape, generator=g, dtype=F64)
            plus = dict(inp, **{k: inp[k] + eps * v})
            minus = dict(inp, **{k: inp[k] - eps * v})
            fd = (f(plus) - f(minus)) / (2 * eps)
            an = float((ag[k] * v).sum())
            assert abs(fd - an) <= 1e-5 * max(1.0, abs(an)), (k, fd, an)


def test_bf16_forward_vjp_equals_autograd():
    """With the forward's bf16 rounding points and exact cotangents, the
    hand-written VJP equals autograd through a straight-through rounding
    (fp64): the bf16 forward structure of the derivative is pinned exactly."""
    T, D, dr, N, chunk = 10, 32, 16, 150, 50
    inp = _inputs(T, D, dr, N, seed=9)
    d_out, d_lb, d_pen = _cot(T, D, 9)
    ag = _autograd(inp, d_out, d_lb, d_pen, chunk, rb=srw_vjp.rb_bf16_straight)
    an = srw_vjp.fused_gate_srw_vjp(**inp, d_out=d_out, d_lb=d_lb, d_pen=d_pen, max_chunk_size=chunk,
                                    rb=srw_vjp.rb_bf16, rc=srw_vjp.rb_exact, dtype=F64)
    keymap = dict(x="dx", h="dh", emb="demb", tau_offset="dtau_offset", read="dread", write="dwrite")
    for k in NAMES:
        a, b = ag[k], an[keymap[k]]
        err = (a - b).abs().max() / a.abs().max().clamp_min(1e-30)
        assert err < 1e-9, (k, float(err))


def test_bf16_cotangents_close_to_exact_cotangents():
    """The reference's bf16 cotangent roundings (same bf16 forward) move each
    gradient by bf16 rounding noise only (relative Frobenius 2e-2)."""
    T, D, dr, N = 16, 64, 32, 400
    inp = _inputs(T, D, dr, N, seed=6)
    d_out, d_lb, d_pen = _cot(T, D, 6)
    ex = srw_vjp.fused_gate_srw_vjp(**inp, d_out=d_out, d_lb=d_lb, d_pen=d_pen, max_chunk_size=200,
                                    rc=srw_vjp.rb_exact, dtype=F64)
    bf = srw_vjp.fused_gate_srw_vjp(**inp, d_out=d_out, d_lb=d_lb, d_pen=d_pen, max_chunk_size=200)
    for k in ("dx", "dh", "demb", "dtau_offset", "dread", "dwrite"):
        a, b = ex[k].float(), bf[k].float()
        rel = float((a - b).norm() / a.norm().clamp_min(1e-30))
        assert rel < 2e-2, (k, rel)


def test_planted_sign_error_is_caught():
    """A VJP with the tau derivative's sign flipped fails the autograd pin."""
    T, D, dr, N = 8, 24, 16, 120
    inp = _inputs(T, D, dr, N, seed=8)
    d_out, d_lb, d_pen = _cot(T, D, 8)
    ag = _autograd(inp, d_out, d_lb, d_pen, 60)
    an = srw_vjp.fused_gate_srw_vjp(**inp, d_out=d_out, d_lb=d_lb, d_pen=d_pen, max_chunk_size=60,
                                    rb=srw_vjp.rb_exact, dtype=F64)
    bad = -an["dtau_offset"]
    assert not torch.allclose(bad, ag["tau_offset"], rtol=1e-6, atol=1e-9)
    assert torch.allclose(an["dtau_offset"], ag["tau_offset"], rtol=1e-9, atol=1e-12)
