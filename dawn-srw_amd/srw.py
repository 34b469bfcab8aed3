"""Drop-in mirror of the reference SRW operator interface.

Reference (madst0614/DAWN-SRW, models/dawn_spatial_v41_exp.py):

* ``make_sharded_srw(mesh, max_chunk_size=2048, dead_threshold=0.01,
  sharpness=..., activation_threshold=..., activation_cutoff=...,
  epsilon=..., max_intensity=...)`` (:352-637) returns
  ``fused_gate_srw(x, h, emb, tau_offset, read, write)`` -> 22-tuple.
* ``make_sharded_srw_paired(...)`` (:640-909) returns the paired QK form
  (h [B,S,2,dr], tau_offset [B,S,2,1], out [B,S,2,D]).
* ``_srw_inference(x, h, emb_norm, tau_offset, w_read, w_write)``
  (:1713-1738) -> out (dtype-preserving, two-pass centred std).
* The v4.0.1 ``make_sharded_srw(mesh, max_chunk_size=2048)`` and
  ``make_sharded_srw_paired`` (models/legacy/dawn_spatial_v401_exp.py:
  194-554, GELU gate) as ``make_sharded_srw_v401`` /
  ``make_sharded_srw_paired_v401`` -> 16-tuple.

The factories return functions with the same positional signature and the
same 22-tuple order, so they slot into ``sharded_fns = (fused_single,
fused_paired)`` (consumed at :1034 and :1164).  The mesh is one device: a
``mesh`` whose ``shape`` has data or model axes larger than 1 is refused
(one GPU; the cross-device psums of the reference are identities there).

Inputs are torch tensors on a HIP device.  Like the reference, the fused
functions cast x, h, emb, read and write to bf16 (:423-430) and return
``out`` as float32 holding bf16-rounded values (:586, :630).  The kernel
computes every per-token and per-unit reduction; this module only turns
those [T]- and [N]-sized vectors into the reference's scalars (:588-635).

The fused functions are autograd nodes: out, score_lb and dead_penalty --
the outputs the reference's training loss uses (scripts/train_jax.py:
586-603) -- backpropagate to all six inputs through ``srw_backward``.
"""

from __future__ import annotations

import torch

from .layer import GateConfig, srw_backward, srw_forward
from . import _capi as C

__all__ = ["make_sharded_srw", "make_sharded_srw_paired", "make_sharded_srw_v401",
           "make_sharded_srw_paired_v401", "srw_inference", "chunk_plan", "GateConfig"]

_TD = C.TDIAG_INDEX


def chunk_plan(n_local: int, max_chunk_size: int):
    """(nc, cs) chunk plan of the N axis (v41:416-420)."""
    nc = max(1, n_local // max_chunk_size)
    while n_local % nc != 0 and nc < n_local:
        nc += 1
    return nc, n_local // nc


def _check_mesh(mesh):
    if mesh is None:
        return
    shape = getattr(mesh, "shape", None)
    if shape is None:
        raise TypeError("mesh must be None or expose a .shape mapping")
    for ax in ("data", "model"):
        if int(shape.get(ax, 1)) != 1:
            raise NotImplementedError(
                f"mesh axis '{ax}' = {shape[ax]}: this build runs the SRW layer on one GPU")


def _diag_tuple(res, N, B, S, R, dead_threshold):
    """The reference's diagnostics (v41:588-635 single, :862-907 paired).

    res: kernel outputs with token_diag [T,R,14] and unit_diag [N,2].
    Per-token outputs keep the reference's [B,S,1] shape (route-averaged
    when R == 2, :864-871).
    """
    td = res["token_diag"]
    g = res["gate_sum"]                         # [T,R]
    na = res["n_active"].to(torch.float32)      # [T,R]
    col = lambda k: td[..., _TD[k]]             # noqa: E731
    s_mean, s_std, tau = col("s_mean"), col("s_std"), col("tau")
    n_tot = float(N)

    def per_token(v):                           # [T,R] -> [B,S,1]
        return v.mean(dim=1).reshape(B, S, 1) if R == 2 else v.reshape(B, S, 1)

    active_frac = per_token(na / n_tot)                            # :589 / :863-864
    gate_max = per_token(col("gate_max"))                          # :583 / :871
    strong_frac = per_token(col("n_strong") / n_tot)               # :590
    boundary_frac = per_token(col("n_boundary") / n_tot)           # :592
    z_mean_active = per_token(g / (na + 1e-8))                     # :594 / :869
    active_denom = torch.clamp_min(na, 1.0)                        # :599
    z_lt_075 = (col("n_band075") / active_denom).mean()            # :600-601
    z_lt_030 = (col("n_band030") / active_denom).mean()
    # moments -> skew / kurtosis (:466-474)
    cube_mean = col("sum_s3") / n_tot
    quad_mean = col("sum_s4") / n_tot
    central_third = cube_mean - 3.0 * s_mean * (s_std ** 2) - s_mean ** 3
    skew = (central_third / (s_std ** 3 + 1e-8)).mean()
    central_fourth = (quad_mean - 4.0 * s_mean * cube_mean
                      + 6.0 * (s_mean ** 2) * (s_std ** 2) + 3.0 * s_mean ** 4)
    kurt = (central_fourth / (s_std ** 4 + 1e-8)).mean()
    # per-unit stats: score LB (:445-447, :476-483), dead units (:543-552)
    ud = res["unit_diag"]
    per_neuron = ud[:, 0] / float(B * S * R)
    mean_score = per_neuron.sum() / n_tot
    var_score = (per_neuron ** 2).sum() / n_tot - mean_score ** 2
    score_lb = var_score / (mean_score ** 2 + var_score + 1e-2)
    dead = (ud[:, 1] < dead_threshold).to(torch.float32)
    dead_penalty = (torch.relu(-per_neuron) * dead).sum()
    dead_count = dead.sum()
    # entropy (:611-618)
    gse = torch.clamp_min(g, 1e-6)
    safe = torch.where(g > 1e-6, col("g_log_g"), torch.zeros_like(g))
    ent = -safe / gse + torch.log(gse)
    ent = torch.where(torch.isfinite(ent), ent, torch.zeros_like(ent))
    return (active_frac, gate_max, score_lb, s_std.mean(), g.mean(), na.mean(),
            strong_frac, boundary_frac, z_mean_active, tau.mean(), z_lt_075,
            z_lt_030, skew, na.std(correction=0), ent.mean(),
            col("int_sum").mean(), kurt, dead_penalty, dead_count,
            col("int_max").max(), col("n_int_cap").sum() / float(B * S * R * N))


# Positions in the 22-tuple (v41:630-635).  The training loss differentiates
# out, score_lb and dead_penalty (scripts/train_jax.py:586-603).
_OUT, _SCORE_LB, _DEAD_PENALTY = 0, 3, 18
# Outputs without a gradient: behind stop_gradient in the reference (score_skew
# and score_kurt :466-474, gate_max :583, tau_abs_mean, z_lt_*,
# active_per_token_std, entropy, dead_count, int_max, int_cap_frac, :599-629)
# or piecewise-constant counts (active_frac, active_n_mean, strong_frac,
# boundary_frac).
_NO_GRAD = (1, 2, 6, 7, 8, 10, 11, 12, 13, 14, 15, 17, 19, 20, 21)
_NAMES = ("out", "active_frac", "gate_max", "score_lb", "score_std", "gate_sum_mean",
          "active_n_mean", "strong_frac", "boundary_frac", "z_mean_active", "tau_abs_mean",
          "z_lt_075", "z_lt_030", "skew", "active_per_token_std", "entropy", "intensity_sum_mean",
          "kurt", "dead_penalty", "dead_count", "int_max", "int_cap_frac")


class _FusedSrw(torch.autograd.Function):
    """fused_gate_srw(_paired) as one autograd node: the forward runs
    srw_forward (bf16, one-pass statistics, diagnostics), the backward runs
    srw_backward with the cotangents of out, score_lb and dead_penalty -- the
    VJP that jax.value_and_grad takes through the reference's checkpointed
    scans (v41:434, 489; scripts/train_jax.py:726).  Differentiating any other
    differentiable diagnostic (score_std, the gate and intensity sums,
    z_mean_active) raises NotImplementedError; the rest carry no gradient, as
    in the reference."""

    @staticmethod
    def forward(ctx, x, h, emb, tau_offset, read, write, routes, consts, cs):
        B, S, D = x.shape
        N = emb.shape[0]
        bf = torch.bfloat16
        xb = x.reshape(B * S, D).to(bf).contiguous()
        hb = h.reshape(B * S, routes, h.shape[-1]).to(bf).contiguous()
        tau = tau_offset.reshape(B * S, routes).to(torch.float32).contiguous()
        eb, rdb, wb = (t.to(bf).contiguous() for t in (emb, read, write))
        # the caller's h is x itself (score = x.E^T, one route): pass the one
        # tensor, which lets the kernels hold a single operand in registers
        h_call = xb if (h is x and routes == 1) else hb
        res = srw_forward(xb, h_call, eb, tau, rdb, wb, stats="onepass", consts=consts,
                          chunk_size=cs, diag=True, want_mask=False)
        shape = (B, S, D) if routes == 1 else (B, S, 2, D)
        out = res["out"].reshape(shape).to(torch.float32)
        outs = (out,) + _diag_tuple(res, N, B, S, routes, consts.dead_threshold)
        # the forward's den and unit statistics: the backward takes them
        # instead of recomputing them from the scores
        ctx.save_for_backward(xb, hb, eb, tau, rdb, wb, res["out"], res["den"], res["unit_diag"])
        ctx.meta = (routes, consts, tuple(t.shape for t in (x, h, emb, tau_offset, read, write)),
                    tuple(t.dtype for t in (x, h, emb, tau_offset, read, write)))
        ctx.mark_non_differentiable(*(outs[i] for i in _NO_GRAD))
        ctx.set_materialize_grads(False)
        return outs

    @staticmethod
    def backward(ctx, *grads):
        for i, g in enumerate(grads):
            if g is not None and i not in (_OUT, _SCORE_LB, _DEAD_PENALTY) and i not in _NO_GRAD:
                raise NotImplementedError(
                    f"the gradient through output {i} ({_NAMES[i]}) of the fused SRW layer is not "
                    "implemented; out, score_lb and dead_penalty are differentiable")
        routes, consts, shapes, dtypes = ctx.meta
        xb, hb, eb, tau, rdb, wb, out_b, den, unit_diag = ctx.saved_tensors
        T, D = xb.shape
        d_out = grads[_OUT]
        if d_out is None:
            d_out = torch.zeros(T, routes, D, dtype=torch.float32, device=xb.device)
        else:
            d_out = d_out.reshape(T, routes, D).to(torch.float32).contiguous()
        d_lb = 0.0 if grads[_SCORE_LB] is None else float(grads[_SCORE_LB])
        d_pen = 0.0 if grads[_DEAD_PENALTY] is None else float(grads[_DEAD_PENALTY])
        g = srw_backward(xb, hb, eb, tau, rdb, wb, out_b, d_out, d_lb, d_pen, consts=consts,
                         den=den.reshape(T, routes), unit_diag=unit_diag)
        res = [g[k] for k in ("dx", "dh", "demb", "dtau_offset", "dread", "dwrite")]
        res = [r.reshape(sh).to(dt) for r, sh, dt in zip(res, shapes, dtypes)]
        return (*res, None, None, None)


def _make(routes: int, mesh, max_chunk_size, dead_threshold, sharpness,
          activation_threshold, activation_cutoff, epsilon, max_intensity):
    _check_mesh(mesh)
    consts = GateConfig(float(sharpness), float(activation_threshold),
                        float(activation_cutoff), float(epsilon),
                        float(max_intensity), float(dead_threshold))

    def fused(x, h, emb, tau_offset, read, write):
        _, cs = chunk_plan(emb.shape[0], max_chunk_size)
        return _FusedSrw.apply(x, h, emb, tau_offset, read, write, routes, consts, cs)

    fused.__name__ = "fused_gate_srw" if routes == 1 else "fused_gate_srw_paired"
    return fused


def make_sharded_srw(mesh=None, max_chunk_size=2048, dead_threshold=0.01,
                     sharpness=500.0, activation_threshold=0.5,
                     activation_cutoff=0.01, epsilon=1e-4, max_intensity=10.0):
    """Single-route fused gate + SRW (v41:352-637); see the module docstring."""
    return _make(1, mesh, max_chunk_size, dead_threshold, sharpness,
                 activation_threshold, activation_cutoff, epsilon, max_intensity)


def make_sharded_srw_paired(mesh=None, max_chunk_size=2048, dead_threshold=0.01,
                            sharpness=500.0, activation_threshold=0.5,
                            activation_cutoff=0.01, epsilon=1e-4,
                            max_intensity=10.0):
    """Paired QK fused gate + SRW sharing one x.R^T (v41:640-909)."""
    return _make(2, mesh, max_chunk_size, dead_threshold, sharpness,
                 activation_threshold, activation_cutoff, epsilon, max_intensity)


def _diag_tuple_v401(res, N, B, S, R=1):
    """The v4.0.1 diagnostics (models/legacy/dawn_spatial_v401_exp.py:
    343-367 single, :525-553 paired): [T,R]- and [N]-sized kernel reductions
    -> the reference's 15 values after out.  token_diag's INT_SUM column
    holds the sum of z+ and its band / boundary / strong columns the v4.0.1
    counts (include/srw_amd.h).  Per-token outputs keep the [B,S,1] shape,
    averaged over the routes when R == 2 (:525-538); every scalar is over
    the (token, route) rows."""
    td = res["token_diag"]
    g = res["gate_sum"]                         # [T,R]
    na = res["n_active"].to(torch.float32)
    col = lambda k: td[..., _TD[k]]             # noqa: E731
    s_mean, s_std, tau = col("s_mean"), col("s_std"), col("tau")
    n_tot = float(N)

    def per_token(v):                           # [T,R] -> [B,S,1]
        return v.mean(dim=1).reshape(B, S, 1) if R == 2 else v.reshape(B, S, 1)

    # skewness from the raw third moment (v401:276-279, :455-458)
    cube_mean = col("sum_s3") / n_tot
    central_third = cube_mean - 3.0 * s_mean * (s_std ** 2) - s_mean ** 3
    skew = (central_third / (s_std ** 3 + 1e-8)).mean()
    # score LB: variance of the per-unit mean score over every (token, route)
    # row (v401:257-260, 281-289; :436)
    per_neuron = res["unit_diag"][:, 0] / float(B * S * R)
    mean_score = per_neuron.sum() / n_tot
    var_score = (per_neuron ** 2).sum() / n_tot - mean_score ** 2
    score_lb = var_score / (mean_score ** 2 + var_score + 1e-2)
    # gate entropy (v401:360-363, :545-548)
    gse = g + 1e-8
    ent = -col("g_log_g") / gse + torch.log(gse)
    act_eps = na + 1e-8
    return (per_token(na / n_tot), per_token(col("gate_max")), score_lb, s_std.mean(), g.mean(), na.mean(),
            per_token(col("n_strong") / n_tot), per_token(col("n_boundary") / n_tot),
            per_token(col("int_sum") / act_eps), tau.mean(),
            (col("n_band075") / act_eps).mean(), (col("n_band030") / act_eps).mean(),
            skew, na.std(correction=0), ent.mean())


# Positions in the v4.0.1 16-tuple (v401:364-367).  Its callers' losses use
# out and score_lb (lb_loss, v401:909, 978); outputs behind stop_gradient
# (gate_max, tau_abs_mean, z_lt_*, score_skew, active_per_token_std,
# gate_entropy, v401:276-279, 344-363) and the counts carry no gradient.
_NO_GRAD_V401 = (1, 2, 6, 7, 8, 10, 11, 12, 13, 14, 15)
_NAMES_V401 = _NAMES[:16]


class _FusedSrwV401(torch.autograd.Function):
    """The v4.0.1 fused_gate_srw(_paired) (v401:230-367, :408-554) as one
    autograd node: the forward runs srw_forward (bf16, the GELU gate, one-pass
    statistics, diagnostics), the backward srw_backward with the gate and the
    cotangents of out and score_lb.  Differentiating score_std, the gate sum
    or z_mean_active raises NotImplementedError."""

    @staticmethod
    def forward(ctx, x, h, emb, tau_offset, read, write, routes, cs):
        B, S, D = x.shape
        N = emb.shape[0]
        bf = torch.bfloat16
        xb = x.reshape(B * S, D).to(bf).contiguous()                       # v401:238-242
        hb = h.reshape(B * S, routes, h.shape[-1]).to(bf).contiguous()
        tau = tau_offset.reshape(B * S, routes).to(torch.float32).contiguous()
        eb, rdb, wb = (t.to(bf).contiguous() for t in (emb, read, write))
        h_call = xb if (h is x and routes == 1) else hb
        res = srw_forward(xb, h_call, eb, tau, rdb, wb, gate="gelu_v401", stats="onepass",
                          chunk_size=cs, diag=True, want_mask=False)
        shape = (B, S, D) if routes == 1 else (B, S, 2, D)
        out = res["out"].reshape(shape).to(torch.float32)
        outs = (out,) + _diag_tuple_v401(res, N, B, S, routes)
        ctx.save_for_backward(xb, hb, eb, tau, rdb, wb, res["out"], res["den"], res["unit_diag"])
        ctx.meta = (routes, tuple(t.shape for t in (x, h, emb, tau_offset, read, write)),
                    tuple(t.dtype for t in (x, h, emb, tau_offset, read, write)))
        ctx.mark_non_differentiable(*(outs[i] for i in _NO_GRAD_V401))
        ctx.set_materialize_grads(False)
        return outs

    @staticmethod
    def backward(ctx, *grads):
        for i, g in enumerate(grads):
            if g is not None and i not in (_OUT, _SCORE_LB) and i not in _NO_GRAD_V401:
                raise NotImplementedError(
                    f"the gradient through output {i} ({_NAMES_V401[i]}) of the v4.0.1 fused SRW layer "
                    "is not implemented; out and score_lb are differentiable")
        routes, shapes, dtypes = ctx.meta
        xb, hb, eb, tau, rdb, wb, out_b, den, unit_diag = ctx.saved_tensors
        T, D = xb.shape
        d_out = grads[_OUT]
        if d_out is None:
            d_out = torch.zeros(T, routes, D, dtype=torch.float32, device=xb.device)
        else:
            d_out = d_out.reshape(T, routes, D).to(torch.float32).contiguous()
        d_lb = 0.0 if grads[_SCORE_LB] is None else float(grads[_SCORE_LB])
        g = srw_backward(xb, hb, eb, tau, rdb, wb, out_b, d_out, d_lb, 0.0, gate="gelu_v401",
                         den=den.reshape(T, routes), unit_diag=unit_diag)
        res = [g[k] for k in ("dx", "dh", "demb", "dtau_offset", "dread", "dwrite")]
        res = [r.reshape(sh).to(dt) for r, sh, dt in zip(res, shapes, dtypes)]
        return (*res, None, None)


def _make_v401(routes, mesh, max_chunk_size):
    _check_mesh(mesh)

    def fused(x, h, emb, tau_offset, read, write):
        _, cs = chunk_plan(emb.shape[0], max_chunk_size)                  # v401:231-235
        return _FusedSrwV401.apply(x, h, emb, tau_offset, read, write, routes, cs)

    fused.__name__ = "fused_gate_srw" if routes == 1 else "fused_gate_srw_paired"
    return fused


def make_sharded_srw_v401(mesh=None, max_chunk_size=2048):
    """The v4.0.1 ``make_sharded_srw(mesh, max_chunk_size=2048)``
    (models/legacy/dawn_spatial_v401_exp.py:194-369): returns
    ``fused_gate_srw(x, h, emb, tau_offset, read, write)`` -> the 16-tuple
    (out, active_frac, gate_max, score_lb, score_std, gate_sum, active_n_mean,
    strong_frac, phi_binary_frac, z_mean_active, tau_abs_mean, z_lt_075_frac,
    z_lt_030_frac, score_skew, active_per_token_std, gate_entropy).  Inputs
    cast to bf16 (v401:238-242), one-pass statistics, R and W rows
    forward-normalised per chunk (v401:300-301); out and score_lb
    backpropagate to the six inputs through ``srw_backward``."""
    return _make_v401(1, mesh, max_chunk_size)


def make_sharded_srw_paired_v401(mesh=None, max_chunk_size=2048):
    """The v4.0.1 ``make_sharded_srw_paired(mesh, max_chunk_size=2048)``
    (v401:372-554): h [B,S,2,dr], tau_offset [B,S,2,1] -> the 16-tuple with
    out [B,S,2,D] and the per-token outputs averaged over the two routes;
    x.R^T shared by both routes; differentiable as the single form."""
    return _make_v401(2, mesh, max_chunk_size)


def srw_inference(x, h, emb_norm, tau_offset, w_read, w_write, *,
                  consts: GateConfig = GateConfig(), gate: str = "v41"):
    """``_srw_inference`` (v41:1713-1738; v4.0.1 form v401:1443-1463 with
    gate="gelu_v401").

    Keeps the input dtype (float32 end to end for float32 inputs) and uses
    the two-pass centred std.  x [..., D], h [..., dr], tau_offset [..., 1].
    Returns float32 out [..., D].
    """
    lead = x.shape[:-1]
    D = x.shape[-1]
    T = 1
    for s in lead:
        T *= int(s)
    xx = x.reshape(T, D).contiguous()
    hh = h.reshape(T, 1, h.shape[-1]).to(x.dtype).contiguous()
    tau = tau_offset.reshape(T, 1).to(torch.float32).contiguous()
    res = srw_forward(xx, hh, emb_norm.to(x.dtype).contiguous(), tau,
                      w_read.to(x.dtype).contiguous(), w_write.to(x.dtype).contiguous(),
                      gate=gate, stats="centered", consts=consts, want_mask=False)
    return res["out"].reshape(*lead, D).to(torch.float32)


def srw_inference_with_gates(x, h, emb_norm, tau_offset, w_read, w_write, *,
                             consts: GateConfig = GateConfig()):
    """``_srw_inference_with_gates`` (v41:1741-1769): ``(out, gate_raw,
    gate_norm)`` with out float32 [..., D] as :func:`srw_inference`, gate_raw
    float32 [..., N] (activation x intensity of every unit) and
    gate_norm = gate_raw / max(sum_n gate_raw, 1e-8) (:1760).  The dense
    gate comes from the tiled families' gate epilogue (bf16 widths multiples
    of 64, fp32 multiples of 32), else from the generic kernels.
    """
    lead = x.shape[:-1]
    D = x.shape[-1]
    T = 1
    for s in lead:
        T *= int(s)
    N = emb_norm.shape[0]
    xx = x.reshape(T, D).contiguous()
    hh = h.reshape(T, 1, h.shape[-1]).to(x.dtype).contiguous()
    tau = tau_offset.reshape(T, 1).to(torch.float32).contiguous()
    res = srw_forward(xx, hh, emb_norm.to(x.dtype).contiguous(), tau,
                      w_read.to(x.dtype).contiguous(), w_write.to(x.dtype).contiguous(),
                      stats="centered", consts=consts, want_mask=False, want_gate=True)
    gate_raw = res["gate"].reshape(*lead, N)
    gate_norm = gate_raw / torch.clamp_min(gate_raw.sum(dim=-1, keepdim=True), 1e-8)  # :1760
    return res["out"].reshape(*lead, D).to(torch.float32), gate_raw, gate_norm
