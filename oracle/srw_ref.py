"""Line-by-line PyTorch-CPU restatement of the DAWN-SRW SRW forward.

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.  Never imported by
the product path.

Reference file abbreviations used in citations:
  v41  = models/dawn_spatial_v41_exp.py          (registered model v4.1)
  v401 = models/legacy/dawn_spatial_v401_exp.py  (GELU-gate paper baseline)

bf16 emulation.  The reference's bf16 path casts x, h, E, R, W to bf16
(v41:423-430) and uses XLA bf16 dots, whose products are accumulated in
fp32 and whose outputs are rounded to bf16 (v41:439, 503, 517, 518).
``dot_bf16`` emulates exactly that: fp32 matmul of bf16-exact operands,
then round-to-nearest-even to bf16.  Elementwise bf16*bf16 products
(v41:518 ``gate_bf * xr``) are computed in fp32 and rounded once, which is
what XLA does for a bf16 multiply.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

__all__ = [
    "SHARPNESS", "ACTIVATION_THRESHOLD", "ACTIVATION_CUTOFF", "EPSILON",
    "MAX_INTENSITY", "DEAD_THRESHOLD", "GateConsts", "V41",
    "bf16_round", "dot_bf16", "chunk_plan",
    "gate_v41", "gate_gelu_v401",
    "srw_inference", "srw_inference_with_gates",
    "fused_gate_srw", "fused_gate_srw_paired",
    "srw_inference_gelu_v401", "fused_gate_srw_gelu_v401",
    "fused_gate_srw_gelu_v401_paired",
    "FUSED_OUTPUT_NAMES", "FUSED_V401_OUTPUT_NAMES",
]

# v41:297-301 -- v4.1 gate constants (closure-baked as float32 at v41:379-383)
SHARPNESS = 500.0
ACTIVATION_THRESHOLD = 0.5
ACTIVATION_CUTOFF = 0.01
EPSILON = 1e-4
MAX_INTENSITY = 10.0
# v41:352 -- make_sharded_srw(..., dead_threshold=0.01, ...)
DEAD_THRESHOLD = 0.01

# Order of the 22-tuple returned by fused_gate_srw (v41:630-635).
FUSED_OUTPUT_NAMES = (
    "out", "active_frac", "gate_max", "score_lb", "score_std", "gate_sum",
    "active_n_mean", "strong_frac", "boundary_frac", "z_mean_active",
    "tau_abs_mean", "z_lt_075_frac", "z_lt_030_frac", "score_skew",
    "active_per_token_std", "gate_entropy", "intensity_sum", "score_kurt",
    "dead_penalty", "dead_count", "int_max", "int_cap_frac",
)
# Order of the 16-tuple returned by the v4.0.1 fused function (v401:352-355).
FUSED_V401_OUTPUT_NAMES = FUSED_OUTPUT_NAMES[:16]


@dataclass(frozen=True)
class GateConsts:
    """The closure constants of make_sharded_srw (v41:352-383)."""
    sharpness: float = SHARPNESS
    activation_threshold: float = ACTIVATION_THRESHOLD
    activation_cutoff: float = ACTIVATION_CUTOFF
    epsilon: float = EPSILON
    max_intensity: float = MAX_INTENSITY
    dead_threshold: float = DEAD_THRESHOLD


V41 = GateConsts()

F32 = torch.float32
F64 = torch.float64
BF16 = torch.bfloat16


def bf16_round(t: torch.Tensor) -> torch.Tensor:
    """Round to bf16 (round-to-nearest-even) and return as float32."""
    return t.to(BF16).to(F32)


def dot_bf16(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """``a @ b.T`` for bf16 operands the way an XLA bf16 dot does it.

    Products of bf16 values are exact in fp32; they are accumulated in fp32
    and the result is rounded to bf16 (v41:439, 503, 517).
    """
    assert a.dtype == BF16 and b.dtype == BF16
    return (a.to(F32) @ b.to(F32).T).to(BF16)


def chunk_plan(n_local: int, max_chunk_size: int) -> tuple[int, int]:
    """Chunk count and size of the N axis (v41:416-420)."""
    nc = max(1, n_local // max_chunk_size)
    while n_local % nc != 0 and nc < n_local:
        nc += 1
    return nc, n_local // nc


def _f(x: float, dtype: torch.dtype) -> torch.Tensor:
    """A scalar constant materialised in ``dtype`` (jnp.float32(c))."""
    return torch.tensor(x, dtype=dtype)


def gate_v41(scores_f: torch.Tensor, tau: torch.Tensor,
             c: GateConsts = V41):
    """v4.1 two-stage gate (v41:506-511; also v41:1724-1729).

    Returns (margin, activation, intensity, gate), all in scores_f.dtype.
    """
    dt = scores_f.dtype
    raw = scores_f - tau
    margin = raw - _f(c.activation_threshold, dt)
    activation = torch.sigmoid(_f(c.sharpness, dt) * margin)
    active_margin = torch.clamp_min(margin - _f(c.activation_cutoff, dt), 0.0)
    intensity = _f(c.epsilon, dt) + torch.minimum(
        active_margin, _f(c.max_intensity, dt))
    gate = activation * intensity
    return margin, activation, intensity, gate


def gate_gelu_v401(raw_f: torch.Tensor, s_std: torch.Tensor):
    """v4.0.1 GELU-shaped threshold gate (v401:307-310, v401:1452-1454).

    z = raw / s_std; Phi(z) = 0.5 (1 + erf(z / sqrt 2)); gate = z Phi(z) for
    z > 0, else 0.  Returns (z, phi, gate).
    """
    dt = raw_f.dtype
    z = raw_f / s_std
    phi = 0.5 * (1.0 + torch.erf(z * _f(0.7071067811865476, dt)))
    gate = torch.where(z > 0, z * phi, torch.zeros((), dtype=dt))
    return z, phi, gate


# --------------------------------------------------------------------------
# _srw_inference: unchunked, dtype-preserving twin (v41:1713-1738)
# --------------------------------------------------------------------------

def _matmul_t(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """``a @ b.T`` in the operands' dtype (bf16 emulated as an XLA dot)."""
    if a.dtype == BF16:
        return dot_bf16(a, b)
    return a @ b.T


def _srw_inference_core(x, h, emb, tau_offset, w_read, w_write, c, acc):
    scores = _matmul_t(h, emb)                                   # v41:1717
    scores_f = scores.to(acc)                                    # v41:1718
    s_mean = scores_f.mean(dim=-1, keepdim=True)                 # v41:1719
    s_std = torch.sqrt(torch.mean(torch.square(scores_f - s_mean),
                                  dim=-1, keepdim=True)) + _f(1e-8, acc)  # :1720-1721
    tau = s_mean + tau_offset.to(acc) * s_std                    # v41:1722
    margin, activation, intensity, gate = gate_v41(scores_f, tau, c)  # :1724-1729
    xr = _matmul_t(x, w_read)                                    # v41:1734
    p = gate.to(scores.dtype) * xr                               # v41:1735
    if p.dtype == BF16:
        raw_out = dot_bf16(p, w_write.T.contiguous())
    else:
        raw_out = p @ w_write
    den = torch.clamp_min(intensity.sum(dim=-1, keepdim=True), 1.0)  # v41:1736
    out = raw_out.to(acc) / den                                  # v41:1737
    return out, dict(scores=scores_f, s_mean=s_mean, s_std=s_std, tau=tau,
                     margin=margin, activation=activation,
                     intensity=intensity, gate=gate, den=den)


def srw_inference(x, h, emb, tau_offset, w_read, w_write, consts: GateConsts = V41,
                  acc_dtype: torch.dtype = F32, return_trace: bool = False):
    """``_srw_inference`` (v41:1713-1738).

    Computes in the inputs' dtype; the reference's ``astype(float32)``
    points use ``acc_dtype`` (float32 as in the reference; float64 gives an
    exact-arithmetic version for pinning).  Two-pass centered std with +1e-8
    outside the sqrt; den = max(sum intensity, 1).
    """
    out, tr = _srw_inference_core(x, h, emb, tau_offset, w_read, w_write,
                                  consts, acc_dtype)
    out = out.to(acc_dtype)                                      # v41:1738
    return (out, tr) if return_trace else out


def srw_inference_with_gates(x, h, emb, tau_offset, w_read, w_write,
                             consts: GateConsts = V41, acc_dtype=F32):
    """``_srw_inference_with_gates`` (v41:1741-1769): (out, gate, gate_norm)."""
    out, tr = _srw_inference_core(x, h, emb, tau_offset, w_read, w_write,
                                  consts, acc_dtype)
    gate = tr["gate"]
    gate_norm = gate / torch.clamp_min(gate.sum(dim=-1, keepdim=True), 1e-8)  # :1760
    return out.to(acc_dtype), gate, gate_norm


# --------------------------------------------------------------------------
# fused_gate_srw: chunked bf16 two-pass layer with diagnostics (v41:415-635)
# --------------------------------------------------------------------------

def _unit_means(scores_f, red_axes):
    """Per-unit mean score over every token row: (B, S) single, (B, S,
    route) paired (v41:445, :725) -- the score_lb statistic."""
    return scores_f.mean(dim=red_axes)


def _route_mean(t):
    """[B,S,2,1] -> [B,S,1]: the paired call's per-token diagnostics are the
    mean over the two routes (v41:864-871)."""
    return t.mean(dim=2)


def _cell_count(B, S, R, N):
    """(token, route, unit) cells the intensity-cap fraction is over:
    B*S*2*N for the paired call (v41:900-901)."""
    return float(B * S * R * N)


def _pass1_stats(h_bf, emb_bf, nc, cs, n_total, route_axis: bool, exact: bool = False):
    """Pass 1 (v41:434-483; paired v41:713-763): exact stats over all chunks.

    ``exact``: float64 operands and sums, no bf16 rounding of the scores (the
    exact-arithmetic form the pins compare with brute force)."""
    acc = F64 if exact else F32
    lead = h_bf.shape[:-1]
    z = torch.zeros(*lead, 1, dtype=acc)
    s_sum, sq_sum, cube_sum, quad_sum = z.clone(), z.clone(), z.clone(), z.clone()
    ns_sum = torch.zeros((), dtype=acc)
    ns_sq = torch.zeros((), dtype=acc)
    red_axes = tuple(range(len(lead)))        # (0,1) single, (0,1,2) paired
    for i in range(nc):
        ec = emb_bf[i * cs:(i + 1) * cs]
        scores_f = (h_bf @ ec.T) if exact else dot_bf16(h_bf, ec).to(F32)  # :439-440
        s_sum = s_sum + scores_f.sum(dim=-1, keepdim=True)         # :441
        sq_sum = sq_sum + (scores_f ** 2).sum(dim=-1, keepdim=True)
        cube_sum = cube_sum + (scores_f ** 3).sum(dim=-1, keepdim=True)
        quad_sum = quad_sum + (scores_f ** 4).sum(dim=-1, keepdim=True)
        per_neuron = _unit_means(scores_f, red_axes)               # :445 / :725
        ns_sum = ns_sum + per_neuron.sum()
        ns_sq = ns_sq + (per_neuron ** 2).sum()
    s_mean = s_sum / n_total                                       # :461
    s_std = torch.sqrt(sq_sum / n_total - s_mean ** 2) + _f(1e-8, acc)  # :462
    cube_mean = cube_sum / n_total                                 # :467
    central_third = cube_mean - 3.0 * s_mean * (s_std ** 2) - s_mean ** 3
    score_skew = (central_third / (s_std ** 3 + 1e-8)).mean()      # :469
    quad_mean = quad_sum / n_total                                 # :471
    central_fourth = (quad_mean - 4.0 * s_mean * cube_mean
                      + 6.0 * (s_mean ** 2) * (s_std ** 2) + 3.0 * s_mean ** 4)
    score_kurt = (central_fourth / (s_std ** 4 + 1e-8)).mean()     # :474
    # :477-483 with a 1x1 mesh (psum over one device is the identity)
    mean_score = ns_sum / n_total
    var_score = ns_sq / n_total - mean_score ** 2
    score_lb = var_score / (mean_score ** 2 + var_score + 1e-2)
    return dict(s_mean=s_mean, s_std=s_std, score_skew=score_skew,
                score_kurt=score_kurt, score_lb=score_lb,
                s_sum=s_sum, sq_sum=sq_sum)


def _prepare(x, h, emb, read, write):
    return (h.to(BF16), x.to(BF16), emb.to(BF16), read.to(BF16),
            write.to(BF16))                                        # :423-430


def fused_gate_srw(x, h, emb, tau_offset, read, write, *,
                   max_chunk_size: int = 2048, consts: GateConsts = V41,
                   return_trace: bool = False):
    """``fused_gate_srw`` of make_sharded_srw (v41:415-635), 1x1 mesh.

    x [B,S,D], h [B,S,dr], emb [N,dr], tau_offset [B,S,1], read/write [N,D].
    Returns the 22-tuple in FUSED_OUTPUT_NAMES order.
    """
    c = consts
    N = emb.shape[0]
    nc, cs = chunk_plan(N, max_chunk_size)                        # :416-420
    B, S, D = x.shape
    h_bf, x_bf, emb_bf, read_bf, write_bf = _prepare(x, h, emb, read, write)
    st = _pass1_stats(h_bf, emb_bf, nc, cs, N, route_axis=False)
    s_mean, s_std = st["s_mean"], st["s_std"]
    tau = s_mean + tau_offset.to(F32) * s_std                      # :464

    int_cap_thresh = _f(c.epsilon, F32) + _f(c.max_intensity, F32) - _f(1e-3, F32)  # :487
    z1 = torch.zeros(B, S, 1, dtype=F32)
    out = torch.zeros(B, S, D, dtype=F32)
    wsum, gmax = z1.clone(), torch.full((B, S, 1), -1e9, dtype=F32)
    act_n, strong, phi_bin, zsum = z1.clone(), z1.clone(), z1.clone(), z1.clone()
    z075, z030, glogg = z1.clone(), z1.clone(), z1.clone()
    dead_pen = torch.zeros((), dtype=F32)
    dead_cnt = torch.zeros((), dtype=F32)
    int_max = torch.zeros((), dtype=F32)
    int_cap = torch.zeros((), dtype=F32)
    trace_margin, trace_gate = [], []
    for i in range(nc):                                            # :489-577
        sl = slice(i * cs, (i + 1) * cs)
        ec, rc, wc = emb_bf[sl], read_bf[sl], write_bf[sl]
        scores_f = dot_bf16(h_bf, ec).to(F32)                      # :503-504
        margin, activation, intensity, gate = gate_v41(scores_f, tau, c)  # :506-511
        chunk_int_max = intensity.max()                            # :513
        chunk_int_cap = (intensity >= int_cap_thresh).to(F32).sum()
        gate_bf = gate.to(BF16)                                    # :516
        xr = dot_bf16(x_bf, rc)                                    # :517
        prod = (gate_bf.to(F32) * xr.to(F32)).to(BF16)             # :518 bf16 multiply
        c_out = dot_bf16(prod, wc.T.contiguous()).to(F32)          # :518
        out = out + c_out
        wsum = wsum + gate.sum(dim=-1, keepdim=True)               # :519
        act_n = act_n + (activation > 0.5).to(F32).sum(dim=-1, keepdim=True)
        strong = strong + (activation > 0.9).to(F32).sum(dim=-1, keepdim=True)
        phi_bin = phi_bin + ((activation > 0.1) & (activation < 0.9)).to(F32).sum(
            dim=-1, keepdim=True)                                  # :524
        zsum = zsum + intensity.sum(dim=-1, keepdim=True)          # :527
        z075 = z075 + ((activation > 0.05) & (activation < 0.95)).to(F32).sum(
            dim=-1, keepdim=True)
        z030 = z030 + ((activation > 0.2) & (activation < 0.8)).to(F32).sum(
            dim=-1, keepdim=True)
        glogg = glogg + (gate * torch.log(gate + 1e-8)).sum(dim=-1, keepdim=True)  # :533-534
        max_gate_chunk = gate.amax(dim=(0, 1))                     # :543
        mean_score_chunk = scores_f.mean(dim=(0, 1))               # :544
        dead_mask = (max_gate_chunk < c.dead_threshold).to(F32)    # :548
        dead_pen = dead_pen + (torch.relu(-mean_score_chunk) * dead_mask).sum()
        dead_cnt = dead_cnt + dead_mask.sum()
        gmax = torch.maximum(gmax, gate.amax(dim=-1, keepdim=True))  # :555
        int_max = torch.maximum(int_max, chunk_int_max)
        int_cap = int_cap + chunk_int_cap
        if return_trace:
            trace_margin.append(margin)
            trace_gate.append(gate)

    den = torch.clamp_min(zsum, 1.0)                               # :584
    out_f = (out / den).to(BF16).to(F32)                           # :585-586, :630
    active_frac = act_n / N                                        # :589
    strong_frac = strong / N
    phi_frac = phi_bin / N
    z_mean_active = wsum / (act_n + 1e-8)                          # :594
    active_denom = torch.clamp_min(act_n, 1.0)                     # :599
    z_lt_075_frac = (z075 / active_denom).mean()
    z_lt_030_frac = (z030 / active_denom).mean()
    gate_sum_eps = torch.clamp_min(wsum, 1e-6)                     # :613
    safe_glogg = torch.where(wsum > 1e-6, glogg, torch.zeros((), dtype=F32))
    ent = -safe_glogg / gate_sum_eps + torch.log(gate_sum_eps)
    ent = torch.where(torch.isfinite(ent), ent, torch.zeros((), dtype=F32))
    res = (
        out_f, active_frac, gmax, st["score_lb"], s_std.mean(), wsum.mean(),
        act_n.mean(), strong_frac, phi_frac, z_mean_active, tau.mean(),
        z_lt_075_frac, z_lt_030_frac, st["score_skew"],
        act_n.std(correction=0), ent.mean(), zsum.mean(), st["score_kurt"],
        dead_pen, dead_cnt, int_max, int_cap / float(B * S * N),
    )
    if not return_trace:
        return res
    trace = dict(s_mean=s_mean, s_std=s_std, tau=tau, den=den, gate_sum=wsum,
                 intensity_sum=zsum, n_active=act_n, raw_out=out,
                 margin=torch.cat(trace_margin, dim=-1),
                 gate=torch.cat(trace_gate, dim=-1), nc=nc, cs=cs)
    return res, trace


def fused_gate_srw_paired(x, h, emb, tau_offset, read, write, *,
                          max_chunk_size: int = 2048,
                          consts: GateConsts = V41, return_trace: bool = False):
    """``fused_gate_srw_paired`` (v41:695-907), 1x1 mesh.

    x [B,S,D], h [B,S,2,dr], tau_offset [B,S,2,1].  x @ read.T is computed
    once per chunk and shared by both routes (v41:796).  Returns the 22-tuple
    (out [B,S,2,D]; per-token outputs averaged over the route axis as in
    v41:864-871).
    """
    c = consts
    N = emb.shape[0]
    nc, cs = chunk_plan(N, max_chunk_size)
    B, S, D = x.shape
    R = h.shape[2]
    h_bf, x_bf, emb_bf, read_bf, write_bf = _prepare(x, h, emb, read, write)
    st = _pass1_stats(h_bf, emb_bf, nc, cs, N, route_axis=True)
    s_mean, s_std = st["s_mean"], st["s_std"]
    tau = s_mean + tau_offset.to(F32) * s_std                      # :744

    int_cap_thresh = _f(c.epsilon, F32) + _f(c.max_intensity, F32) - _f(1e-3, F32)
    z1 = torch.zeros(B, S, R, 1, dtype=F32)
    out = torch.zeros(B, S, R, D, dtype=F32)
    wsum, gmax = z1.clone(), torch.full((B, S, R, 1), -1e9, dtype=F32)
    act_n, strong, phi_bin, zsum = z1.clone(), z1.clone(), z1.clone(), z1.clone()
    z075, z030, glogg = z1.clone(), z1.clone(), z1.clone()
    dead_pen = torch.zeros((), dtype=F32)
    dead_cnt = torch.zeros((), dtype=F32)
    int_max = torch.zeros((), dtype=F32)
    int_cap = torch.zeros((), dtype=F32)
    trace_margin, trace_gate = [], []
    for i in range(nc):                                            # :768-840
        sl = slice(i * cs, (i + 1) * cs)
        ec, rc, wc = emb_bf[sl], read_bf[sl], write_bf[sl]
        scores_f = dot_bf16(h_bf, ec).to(F32)                      # :782-783
        margin, activation, intensity, gate = gate_v41(scores_f, tau, c)
        chunk_int_max = intensity.max()
        chunk_int_cap = (intensity >= int_cap_thresh).to(F32).sum()
        gate_bf = gate.to(BF16)                                    # :795
        xr = dot_bf16(x_bf, rc)                                    # :796 (shared)
        prod = (gate_bf.to(F32) * xr.to(F32)[:, :, None, :]).to(BF16)
        c_out = dot_bf16(prod, wc.T.contiguous()).to(F32)          # :797
        out = out + c_out
        wsum = wsum + gate.sum(dim=-1, keepdim=True)
        act_n = act_n + (activation > 0.5).to(F32).sum(dim=-1, keepdim=True)
        strong = strong + (activation > 0.9).to(F32).sum(dim=-1, keepdim=True)
        phi_bin = phi_bin + ((activation > 0.1) & (activation < 0.9)).to(F32).sum(
            dim=-1, keepdim=True)
        zsum = zsum + intensity.sum(dim=-1, keepdim=True)
        z075 = z075 + ((activation > 0.05) & (activation < 0.95)).to(F32).sum(
            dim=-1, keepdim=True)
        z030 = z030 + ((activation > 0.2) & (activation < 0.8)).to(F32).sum(
            dim=-1, keepdim=True)
        glogg = glogg + (gate * torch.log(gate + 1e-8)).sum(dim=-1, keepdim=True)
        max_gate_chunk = gate.amax(dim=(0, 1, 2))                  # :817
        mean_score_chunk = scores_f.mean(dim=(0, 1, 2))            # :818
        dead_mask = (max_gate_chunk < c.dead_threshold).to(F32)
        dead_pen = dead_pen + (torch.relu(-mean_score_chunk) * dead_mask).sum()
        dead_cnt = dead_cnt + dead_mask.sum()
        gmax = torch.maximum(gmax, gate.amax(dim=-1, keepdim=True))
        int_max = torch.maximum(int_max, chunk_int_max)
        int_cap = int_cap + chunk_int_cap
        if return_trace:
            trace_margin.append(margin)
            trace_gate.append(gate)

    den = torch.clamp_min(zsum, 1.0)                               # :858
    out_f = (out / den).to(BF16).to(F32)                           # :859-860
    active_frac = act_n / N
    z_mean_active = wsum / (act_n + 1e-8)                          # :869
    active_denom = torch.clamp_min(act_n, 1.0)
    gate_sum_eps = torch.clamp_min(wsum, 1e-6)
    safe_glogg = torch.where(wsum > 1e-6, glogg, torch.zeros((), dtype=F32))
    ent = -safe_glogg / gate_sum_eps + torch.log(gate_sum_eps)
    ent = torch.where(torch.isfinite(ent), ent, torch.zeros((), dtype=F32))
    res = (
        out_f, _route_mean(active_frac), _route_mean(gmax), st["score_lb"],
        s_std.mean(), wsum.mean(), act_n.mean(), _route_mean(strong / N),
        _route_mean(phi_bin / N), _route_mean(z_mean_active), tau.mean(),
        (z075 / active_denom).mean(), (z030 / active_denom).mean(),
        st["score_skew"], act_n.std(correction=0), ent.mean(), zsum.mean(),
        st["score_kurt"], dead_pen, dead_cnt, int_max,
        int_cap / _cell_count(B, S, R, N),                         # :900-901
    )
    if not return_trace:
        return res
    trace = dict(s_mean=s_mean, s_std=s_std, tau=tau, den=den, gate_sum=wsum,
                 intensity_sum=zsum, n_active=act_n, raw_out=out,
                 margin=torch.cat(trace_margin, dim=-1),
                 gate=torch.cat(trace_gate, dim=-1), nc=nc, cs=cs)
    return res, trace


# --------------------------------------------------------------------------
# v4.0.1 GELU gate (legacy paper baseline)
# --------------------------------------------------------------------------

def _norm_rows(t: torch.Tensor) -> torch.Tensor:
    """r / (||r|| + 1e-8) in t's dtype (v401:300-301, v401:1456-1457)."""
    if t.dtype == BF16:
        nrm = torch.linalg.vector_norm(t.to(F32), dim=-1, keepdim=True).to(BF16)
        return (t.to(F32) / (nrm + _f(1e-8, BF16)).to(F32)).to(BF16)
    return t / (torch.linalg.vector_norm(t, dim=-1, keepdim=True) + 1e-8)


def srw_inference_gelu_v401(x, h, emb, tau_offset, w_read, w_write,
                            acc_dtype: torch.dtype = F32, return_trace=False):
    """v4.0.1 ``_srw_inference`` (v401:1443-1463): GELU gate, den = max(sum gate, 1)."""
    scores = _matmul_t(h, emb)
    scores_f = scores.to(acc_dtype)
    s_mean = scores_f.mean(dim=-1, keepdim=True)
    s_std = torch.sqrt(torch.mean(torch.square(scores_f - s_mean),
                                  dim=-1, keepdim=True)) + _f(1e-8, acc_dtype)
    tau = s_mean + tau_offset.to(acc_dtype) * s_std
    raw = (scores - tau.to(scores.dtype)).to(acc_dtype)            # :1451-1452
    z, phi, gate = gate_gelu_v401(raw, s_std)
    r_n = _norm_rows(w_read)
    w_n = _norm_rows(w_write)
    xr = _matmul_t(x, r_n)
    p = gate.to(scores.dtype) * xr
    if p.dtype == BF16:
        raw_out = dot_bf16(p, w_n.T.contiguous())
    else:
        raw_out = p @ w_n
    den = torch.clamp_min(gate.sum(dim=-1, keepdim=True), 1.0)     # :1461-1462
    out = (raw_out.to(acc_dtype) / den).to(acc_dtype)
    if return_trace:
        return out, dict(scores=scores_f, s_mean=s_mean, s_std=s_std, tau=tau,
                         z=z, gate=gate, den=den)
    return out


def _v401_den(gate_sum: torch.Tensor, zpos_sum: torch.Tensor) -> torch.Tensor:
    """den = max(sum gate, 1) (v401:340: the psum of total_weighted_cost,
    the chunk sums of gate at :310).  ``zpos_sum`` (sum of z+, the
    z_mean_active numerator) is not part of it."""
    return torch.clamp_min(gate_sum, 1.0)


def fused_gate_srw_gelu_v401(x, h, emb, tau_offset, read, write, *,
                             max_chunk_size: int = 2048, return_trace=False,
                             exact: bool = False):
    """v4.0.1 ``fused_gate_srw`` (v401:230-367), 1x1 mesh -> 16-tuple.

    Pass 1 as v4.1 but without the 4th moment (v401:246-284).  Pass 2
    forward-normalises each chunk's R and W rows in bf16 (v401:300-301),
    gates with z Phi(z) (v401:303-306), den = max(sum gate, 1) (v401:340).

    ``exact``: the same steps in float64 with no bf16 rounding anywhere (the
    operands are widened, not rounded): the exact-arithmetic form the oracle
    pins compare with the brute-force loop and with
    ``srw_inference_gelu_v401``.
    """
    N = emb.shape[0]
    nc, cs = chunk_plan(N, max_chunk_size)                         # v401:231-235
    B, S, D = x.shape
    acc = F64 if exact else F32
    if exact:
        h_bf, x_bf, emb_bf, read_bf, write_bf = (t.to(F64) for t in (h, x, emb, read, write))
        dot = lambda a, b: a @ b.T                                 # noqa: E731
        rnd = lambda t: t                                          # noqa: E731
    else:
        h_bf, x_bf, emb_bf, read_bf, write_bf = _prepare(x, h, emb, read, write)  # v401:238-242
        # operands held as float32 are bf16-exact here (rounded by ``rnd``)
        dot = lambda a, b: dot_bf16(a.to(BF16), b.to(BF16)).to(F32)  # noqa: E731
        rnd = bf16_round
    st = _pass1_stats(h_bf, emb_bf, nc, cs, N, route_axis=False, exact=exact)
    s_mean, s_std = st["s_mean"], st["s_std"]
    tau = s_mean + tau_offset.to(acc) * s_std                      # v401:274
    z1 = torch.zeros(B, S, 1, dtype=acc)
    out = torch.zeros(B, S, D, dtype=acc)
    wsum, gmax = z1.clone(), torch.full((B, S, 1), -1e9, dtype=acc)
    act_n, strong, phi_bin, zsum = z1.clone(), z1.clone(), z1.clone(), z1.clone()
    z075, z030, glogg = z1.clone(), z1.clone(), z1.clone()
    trace_z, trace_gate = [], []
    for i in range(nc):                                            # v401:286-335
        sl = slice(i * cs, (i + 1) * cs)
        ec = emb_bf[sl]
        rc = _norm_rows(read_bf[sl])                               # v401:300
        wc = _norm_rows(write_bf[sl])                              # v401:301
        scores = dot(h_bf, ec)                                     # v401:302 (bf16 dot output)
        raw = scores - tau                                         # v401:303
        z, phi, gate = gate_gelu_v401(raw, s_std)                  # v401:304-306
        gate_bf = rnd(gate)                                        # v401:307
        xr = dot(x_bf, rc)                                         # v401:308
        prod = rnd(gate_bf * xr)                                   # v401:309 bf16 multiply
        out = out + dot(prod, wc.T.contiguous())                   # v401:309 bf16 dot, as f32
        wsum = wsum + gate.sum(dim=-1, keepdim=True)               # v401:310
        act_n = act_n + (gate > 0.0).to(acc).sum(dim=-1, keepdim=True)
        strong = strong + (gate > 0.5).to(acc).sum(dim=-1, keepdim=True)
        phi_bin = phi_bin + ((phi > 0.95) | (phi < 0.05)).to(acc).sum(dim=-1, keepdim=True)
        zsum = zsum + torch.where(z > 0, z, torch.zeros((), dtype=acc)).sum(
            dim=-1, keepdim=True)                                  # v401:314
        z075 = z075 + ((z > 0) & (z < 0.75)).to(acc).sum(dim=-1, keepdim=True)
        z030 = z030 + ((z > 0) & (z < 0.30)).to(acc).sum(dim=-1, keepdim=True)
        glogg = glogg + (gate * torch.log(gate + 1e-8)).sum(dim=-1, keepdim=True)  # v401:317-318
        gmax = torch.maximum(gmax, gate.amax(dim=-1, keepdim=True))
        if return_trace:
            trace_z.append(z)
            trace_gate.append(gate)
    den = _v401_den(wsum, zsum)                                    # v401:340
    out_f = rnd(out / den)                                         # v401:341-342
    gate_sum_eps = wsum + 1e-8                                     # v401:361
    ent = -glogg / gate_sum_eps + torch.log(gate_sum_eps)
    res = (
        out_f, act_n / N, gmax, st["score_lb"], s_std.mean(), wsum.mean(),
        act_n.mean(), strong / N, phi_bin / N, zsum / (act_n + 1e-8), tau.mean(),
        (z075 / (act_n + 1e-8)).mean(), (z030 / (act_n + 1e-8)).mean(),
        st["score_skew"], act_n.std(correction=0), ent.mean(),
    )
    if not return_trace:
        return res
    return res, dict(s_mean=s_mean, s_std=s_std, tau=tau, den=den,
                     gate_sum=wsum, n_active=act_n, raw_out=out,
                     z=torch.cat(trace_z, dim=-1), gate=torch.cat(trace_gate, dim=-1),
                     nc=nc, cs=cs)


def fused_gate_srw_gelu_v401_paired(x, h, emb, tau_offset, read, write, *,
                                    max_chunk_size: int = 2048, return_trace=False,
                                    exact: bool = False):
    """v4.0.1 ``fused_gate_srw_paired`` (v401:408-554), 1x1 mesh -> 16-tuple.

    x [B,S,D], h [B,S,2,dr], tau_offset [B,S,2,1].  Statistics per (token,
    route) row (v401:426-457); x @ R_norm^T once per chunk, shared by both
    routes (v401:496-497); per-token outputs averaged over the route axis
    (v401:532-541); every scalar over (B, S, 2), per-unit score means over
    (B, S, 2) for score_lb (v401:436).  ``exact`` as in
    ``fused_gate_srw_gelu_v401``.
    """
    N = emb.shape[0]
    nc, cs = chunk_plan(N, max_chunk_size)                         # v401:409-413
    B, S, D = x.shape
    R = h.shape[2]
    acc = F64 if exact else F32
    if exact:
        h_bf, x_bf, emb_bf, read_bf, write_bf = (t.to(F64) for t in (h, x, emb, read, write))
        dot = lambda a, b: a @ b.T                                 # noqa: E731
        rnd = lambda t: t                                          # noqa: E731
    else:
        h_bf, x_bf, emb_bf, read_bf, write_bf = _prepare(x, h, emb, read, write)  # v401:416-420
        dot = lambda a, b: dot_bf16(a.to(BF16), b.to(BF16)).to(F32)  # noqa: E731
        rnd = bf16_round
    st = _pass1_stats(h_bf, emb_bf, nc, cs, N, route_axis=True, exact=exact)
    s_mean, s_std = st["s_mean"], st["s_std"]                      # [B,S,2,1]
    tau = s_mean + tau_offset.to(acc) * s_std                      # v401:453
    z1 = torch.zeros(B, S, R, 1, dtype=acc)
    out = torch.zeros(B, S, R, D, dtype=acc)
    wsum, gmax = z1.clone(), torch.full((B, S, R, 1), -1e9, dtype=acc)
    act_n, strong, phi_bin, zsum = z1.clone(), z1.clone(), z1.clone(), z1.clone()
    z075, z030, glogg = z1.clone(), z1.clone(), z1.clone()
    trace_z, trace_gate = [], []
    for i in range(nc):                                            # v401:471-514
        sl = slice(i * cs, (i + 1) * cs)
        ec = emb_bf[sl]
        rc = _norm_rows(read_bf[sl])                               # v401:479
        wc = _norm_rows(write_bf[sl])                              # v401:480
        scores = dot(h_bf, ec)                                     # v401:481 [B,S,2,cs]
        raw = scores - tau                                         # v401:482
        z, phi, gate = gate_gelu_v401(raw, s_std)                  # v401:483-485
        gate_bf = rnd(gate)                                        # v401:486
        xr = dot(x_bf, rc)                                         # v401:487 [B,S,cs], shared
        prod = rnd(gate_bf * xr[:, :, None, :])                    # v401:488 bf16 multiply
        out = out + dot(prod, wc.T.contiguous())                   # v401:488 bf16 dot, as f32
        wsum = wsum + gate.sum(dim=-1, keepdim=True)               # v401:489
        act_n = act_n + (gate > 0.0).to(acc).sum(dim=-1, keepdim=True)
        strong = strong + (gate > 0.5).to(acc).sum(dim=-1, keepdim=True)
        phi_bin = phi_bin + ((phi > 0.95) | (phi < 0.05)).to(acc).sum(dim=-1, keepdim=True)
        zsum = zsum + torch.where(z > 0, z, torch.zeros((), dtype=acc)).sum(dim=-1, keepdim=True)
        z075 = z075 + ((z > 0) & (z < 0.75)).to(acc).sum(dim=-1, keepdim=True)
        z030 = z030 + ((z > 0) & (z < 0.30)).to(acc).sum(dim=-1, keepdim=True)
        glogg = glogg + (gate * torch.log(gate + 1e-8)).sum(dim=-1, keepdim=True)  # v401:496-497
        gmax = torch.maximum(gmax, gate.amax(dim=-1, keepdim=True))
        if return_trace:
            trace_z.append(z)
            trace_gate.append(gate)
    den = _v401_den(wsum, zsum)                                    # v401:521-522, per route
    out_f = rnd(out / den)                                         # v401:523-524
    act_eps = act_n + 1e-8
    gate_sum_eps = wsum + 1e-8                                     # v401:546
    ent = -glogg / gate_sum_eps + torch.log(gate_sum_eps)
    res = (
        out_f, _route_mean(act_n / N), _route_mean(gmax), st["score_lb"], s_std.mean(),
        wsum.mean(), act_n.mean(), _route_mean(strong / N), _route_mean(phi_bin / N),
        _route_mean(zsum / act_eps), tau.mean(),                   # v401:526-543
        (z075 / act_eps).mean(), (z030 / act_eps).mean(),
        st["score_skew"], act_n.std(correction=0), ent.mean(),
    )
    if not return_trace:
        return res
    return res, dict(s_mean=s_mean, s_std=s_std, tau=tau, den=den,
                     gate_sum=wsum, n_active=act_n, raw_out=out,
                     z=torch.cat(trace_z, dim=-1), gate=torch.cat(trace_gate, dim=-1),
                     nc=nc, cs=cs)
