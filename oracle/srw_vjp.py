"""Restatement of the SRW layer's reverse-mode derivative (VJP).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.  Never imported by
the product path.

The reference trains through ``fused_gate_srw`` (models/dawn_spatial_v41_exp.py
:415-635) with ``jax.value_and_grad`` (scripts/train_jax.py:726); its VJP is
whatever JAX autodiff makes of the forward (the two scans are
``jax.checkpoint``-ed, :434 / :489, so the backward recomputes the forward).
Three of the 22 outputs enter the training loss (scripts/train_jax.py:
586-603): ``out`` (through the cross-entropy), ``score_lb`` (``lb_weight *
aux_loss``) and ``dead_penalty`` (``dead_penalty_weight * dead_penalty``);
the others are observational (several behind ``stop_gradient``).

This module restates, for one route (rows = tokens):

* ``fused_terms`` -- the forward of those three outputs, with every bf16
  rounding point of the reference behind a rounding function ``rb`` (bf16
  round-to-nearest-even, or the identity for exact-arithmetic pinning);
* ``fused_gate_srw_vjp`` -- their VJP written out by hand, in the same
  precision structure: cotangents of bf16 values are rounded to bf16 where
  JAX's transpose rules produce bf16 (the transposes of the bf16 casts and
  of the bf16 dots and products), f32 elsewhere.

Pinning (tests/test_backward_oracle.py): ``fused_terms`` (bf16) equals the
full forward restatement ``srw_ref.fused_gate_srw`` on out / score_lb /
dead_penalty; the exact-arithmetic VJP equals torch autograd of the exact
``fused_terms`` (fp64) to 1e-9; autograd agrees with central finite
differences (fp64); with the bf16 forward and exact cotangents the VJP
equals autograd through a straight-through rounding (fp64, 1e-9); the bf16
cotangent roundings themselves move each gradient by 0.3-0.5% (bounded at
2e-2).  Those roundings and XLA's accumulation orders (per chunk, where two
cotangent paths meet) are third-party behaviour no vector fixes: bit-level
agreement with the reference's gradients is parity unpinned.
"""

from __future__ import annotations

import torch

from oracle.srw_ref import V41, GateConsts, chunk_plan

F32 = torch.float32
F64 = torch.float64
BF16 = torch.bfloat16

__all__ = ["fused_terms", "fused_gate_srw_vjp", "rb_bf16", "rb_exact", "rb_bf16_straight"]


def rb_bf16(t: torch.Tensor) -> torch.Tensor:
    """Round to bf16 (RNE) and return in the tensor's own dtype."""
    return t.to(BF16).to(t.dtype)


def rb_exact(t: torch.Tensor) -> torch.Tensor:
    return t


def rb_bf16_straight(t: torch.Tensor) -> torch.Tensor:
    """bf16 rounding in the forward, identity in autograd's backward: the
    forward of ``rb_bf16`` with exact cotangents."""
    return t + (rb_bf16(t) - t).detach()


def _consts(c: GateConsts, dt):
    f = lambda v: torch.tensor(v, dtype=dt)  # noqa: E731
    return (f(c.sharpness), f(c.activation_threshold), f(c.activation_cutoff),
            f(c.epsilon), f(c.max_intensity), c.dead_threshold)


def _forward(x, h, emb, tau_offset, read, write, c, max_chunk_size, rb, dt):
    """Shared forward (v41:423-586, one route, 1x1 mesh); returns the three
    outputs and the intermediates the VJP needs."""
    sharp, thr, cut, eps, maxi, dead_thr = _consts(c, dt)
    T, D = x.shape
    N = emb.shape[0]
    nc, cs = chunk_plan(N, max_chunk_size)                           # :416-420
    hb, xb, eb, rdb, wb = (rb(t.to(dt)) for t in (h, x, emb, read, write))  # :423-430
    s = rb(hb @ eb.T)                                                # :439-440 / :503-504
    mean = s.sum(dim=-1, keepdim=True) / N                           # :441, :461
    sq = (s * s).sum(dim=-1, keepdim=True) / N                       # :442
    var = sq - mean * mean
    std = torch.sqrt(var) + 1e-8                                     # :462
    tau = mean + tau_offset.to(dt) * std                             # :464
    m = s - tau - thr                                                # :506-507
    act = torch.sigmoid(sharp * m)                                   # :508
    am = torch.clamp_min(m - cut, 0.0)                               # :509
    it = eps + torch.minimum(am, maxi)                               # :510
    g = act * it                                                     # :511
    gb = rb(g)                                                       # :516
    xr = rb(xb @ rdb.T)                                              # :517
    p = rb(gb * xr)                                                  # :518 bf16 multiply
    raw = torch.zeros(T, D, dtype=dt)
    for k in range(nc):                                              # chunk scan :489-577
        sl = slice(k * cs, (k + 1) * cs)
        raw = raw + rb(p[:, sl] @ wb[sl])                            # :518 bf16 dot per chunk
    zsum = it.sum(dim=-1, keepdim=True)                              # :527
    den = torch.clamp_min(zsum, 1.0)                                 # :584
    out = rb(raw / den)                                              # :585-586
    # score_lb (:445-447, :477-483): variance of the per-unit mean score
    pn = s.mean(dim=0)                                               # [N]
    ms = pn.sum() / N
    vs = (pn * pn).sum() / N - ms * ms
    lb = vs / (ms * ms + vs + 1e-2)
    # dead penalty (:543-552): max gate per unit behind stop_gradient
    dead = (g.detach().amax(dim=0) < dead_thr).to(dt)
    pen = (torch.relu(-pn) * dead).sum()
    inter = dict(hb=hb, xb=xb, eb=eb, rdb=rdb, wb=wb, s=s, mean=mean, var=var, std=std,
                 tau=tau, m=m, act=act, am=am, it=it, g=g, gb=gb, xr=xr, p=p, raw=raw,
                 zsum=zsum, den=den, pn=pn, ms=ms, vs=vs, dead=dead, nc=nc, cs=cs,
                 consts=(sharp, thr, cut, eps, maxi))
    return (out, lb, pen), inter


def fused_terms(x, h, emb, tau_offset, read, write, *, consts: GateConsts = V41,
                max_chunk_size: int = 2048, rb=rb_bf16, dtype=F32):
    """(out [T, D], score_lb, dead_penalty) of fused_gate_srw for one route.

    x [T, D], h [T, dr], emb [N, dr], tau_offset [T, 1], read / write [N, D].
    Differentiable with torch autograd (the dead mask is detached as the
    reference's stop_gradient, v41:545-549).
    """
    terms, _ = _forward(x, h, emb, tau_offset, read, write, consts, max_chunk_size, rb, dtype)
    return terms


def fused_gate_srw_vjp(x, h, emb, tau_offset, read, write, d_out, d_lb=0.0, d_pen=0.0, *,
                       consts: GateConsts = V41, max_chunk_size: int = 2048,
                       rb=rb_bf16, rc=None, dtype=F32) -> dict:
    """Gradients of <d_out, out> + d_lb * score_lb + d_pen * dead_penalty with
    respect to x, h, emb, tau_offset, read and write (all returned in
    ``dtype``), for one route.  ``rb`` rounds the forward's bf16 values,
    ``rc`` (default: ``rb``) the cotangents at the reference's bf16
    transposes.  With both ``rb_exact`` in fp64 this is the exact derivative
    of ``fused_terms``; with ``rb=rb_bf16, rc=rb_exact`` it is the derivative
    of the bf16 forward with exact cotangents.
    """
    dt = dtype
    fwd_rb = rb
    rb = rc if rc is not None else fwd_rb  # below: cotangent roundings
    (out, lb, pen), v = _forward(x, h, emb, tau_offset, read, write, consts, max_chunk_size, fwd_rb, dt)
    sharp, thr, cut, eps, maxi = v["consts"]
    T, D = x.shape
    N = emb.shape[0]
    s, act, it, g, gb, xr, p = v["s"], v["act"], v["it"], v["g"], v["gb"], v["xr"], v["p"]
    den, zsum = v["den"], v["zsum"]

    # out = rb(raw / den): the cotangent of the bf16 cast is rounded to bf16
    dq = rb(d_out.to(dt))
    draw = dq / den
    dden = -(dq * v["raw"]).sum(dim=-1, keepdim=True) / (den * den)
    dden = torch.where(zsum > 1.0, dden, torch.zeros_like(dden))     # max(., 1) (:584)
    # raw = sum_k rb(p_k @ W_k): each chunk's cotangent is rb(draw) (astype f32 transpose)
    drb = rb(draw)
    dp = torch.empty_like(p)
    dW = torch.empty(N, D, dtype=dt)
    for k in range(v["nc"]):
        sl = slice(k * v["cs"], (k + 1) * v["cs"])
        dp[:, sl] = rb(drb @ v["wb"][sl].T)                           # bf16 dot transpose
        dW[sl] = rb(p[:, sl].T @ drb)
    # p = rb(gb * xr): bf16 multiply transposes
    dgb = rb(dp * xr)
    dxr = rb(dp * gb)
    dg = dgb                                                          # gb = rb(g): f32 cotangent
    # g = act * it; it = eps + min(am, maxi); am = max(m - cut, 0); act = sigmoid(sharp m)
    dact = dg * it
    dit = dg * act + dden                                             # den = max(sum it, 1)
    dam = torch.where(v["am"] < maxi, dit, torch.zeros_like(dit))
    dm = torch.where(v["m"] - cut > 0, dam, torch.zeros_like(dam))
    dm = dm + dact * sharp * act * (1.0 - act)
    # m = s - tau - thr; tau = mean + off * std; std = sqrt(sq - mean^2) + 1e-8
    dtau = -dm.sum(dim=-1, keepdim=True)
    doff = dtau * v["std"]
    dstd = dtau * tau_offset.to(dt)
    dvar = dstd / (2.0 * torch.sqrt(v["var"]))
    dmean = dtau - 2.0 * v["mean"] * dvar
    ds = dm + dmean / N + (2.0 / N) * dvar * s
    # score_lb and the dead penalty through the per-unit mean scores pn = mean_t s
    pn, ms, vs = v["pn"], v["ms"], v["vs"]
    Z = ms * ms + vs + 1e-2
    dlb_dvs = (ms * ms + 1e-2) / (Z * Z)
    dlb_dms = -2.0 * ms * vs / (Z * Z)
    dpn = d_lb * (dlb_dvs * (2.0 * pn - 2.0 * ms) / N + dlb_dms / N)
    dpn = dpn + d_pen * torch.where(pn < 0, -v["dead"], torch.zeros_like(pn))
    ds = ds + dpn[None, :] / T
    # s = rb(hb @ eb^T), xr = rb(xb @ rdb^T): bf16 cotangents into bf16 dots
    dsb = rb(ds)
    dh = rb(dsb @ v["eb"])
    demb = rb(dsb.T @ v["hb"])
    dx = rb(dxr @ v["rdb"])
    dread = rb(dxr.T @ v["xb"])
    return dict(dx=dx, dh=dh, demb=demb, dtau_offset=doff, dread=dread, dwrite=dW,
                out=out, score_lb=lb, dead_penalty=pen, den=den, tau=v["tau"])
