"""Host-side assembly of the drop-in's diagnostics tuples (CPU, no GPU).

The v4.0.1 fused function's 16-tuple (models/legacy/dawn_spatial_v401_exp.py:
343-367) is formed in ``srw._diag_tuple_v401`` from the kernels' per-token
columns (token_diag) and per-unit sums (unit_diag).  Here those columns are
computed in float64 from the exact-arithmetic oracle's scores and gates --
the oracle whose 16-tuple tests/test_oracle_pins.py pins against numpy /
scipy closed forms -- and the assembled tuple must equal the oracle's.  One
token has no unit above its threshold, so that the entropy's +1e-8 guard
(v401:361) and the z-band denominators (v401:349-353) are exercised where
other guards (clamps, finite filters) would give other values.
"""

from __future__ import annotations

import math

import torch

from oracle import srw_ref

F64 = torch.float64


def _inputs(B, S, D, dr, N, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, S, D, generator=g, dtype=F64)
    h = torch.randn(B, S, dr, generator=g, dtype=F64)
    e = torch.randn(N, dr, generator=g, dtype=F64)
    e = e / e.norm(dim=-1, keepdim=True)
    r = torch.randn(N, D, generator=g, dtype=F64)
    w = torch.randn(N, D, generator=g, dtype=F64)
    tau = torch.empty(B, S, 1, dtype=F64).uniform_(-0.6, 1.2, generator=g)
    tau[0, 1, 0] = 50.0                      # no unit passes: gate_sum 0, n_active 0
    return x, h, e, tau, r, w


def _kernel_columns(tr, h, e, B, S, N):
    """token_diag / unit_diag / gate_sum / n_active as the kernels define
    them (include/srw_amd.h), from the oracle's trace, in float64."""
    T = B * S
    z = tr["z"].reshape(T, N)
    gate = tr["gate"].reshape(T, N)
    s_std = tr["s_std"].reshape(T)
    tau = tr["tau"].reshape(T)
    scores = (h.reshape(T, -1) @ e.T)                          # the exact scores
    phi = 0.5 * (1.0 + torch.erf(z / math.sqrt(2.0)))
    td = torch.zeros(T, 1, 14, dtype=F64)
    td[:, 0, 0] = tr["s_mean"].reshape(T)
    td[:, 0, 1] = s_std
    td[:, 0, 2] = tau
    td[:, 0, 3] = (scores ** 3).sum(-1)
    td[:, 0, 4] = (scores ** 4).sum(-1)
    td[:, 0, 5] = gate.amax(-1)
    td[:, 0, 6] = z.clamp_min(0.0).sum(-1)                     # sum of z+
    td[:, 0, 7] = (gate > 0.5).sum(-1)
    td[:, 0, 8] = ((phi > 0.95) | (phi < 0.05)).sum(-1)
    td[:, 0, 9] = ((z > 0) & (z < 0.75)).sum(-1)
    td[:, 0, 10] = ((z > 0) & (z < 0.30)).sum(-1)
    td[:, 0, 11] = (gate * torch.log(gate + 1e-8)).sum(-1)
    ud = torch.stack([scores.sum(0), gate.amax(0)], dim=-1)
    return dict(token_diag=td, unit_diag=ud, gate_sum=gate.sum(-1).reshape(T, 1),
                n_active=(gate > 0).sum(-1).reshape(T, 1).to(torch.int32))


def test_v401_16_tuple_assembly_matches_oracle(pkg):
    B, S, D, dr, N = 2, 6, 12, 8, 90
    x, h, e, tau, r, w = _inputs(B, S, D, dr, N, seed=71)
    ref, tr = srw_ref.fused_gate_srw_gelu_v401(x, h, e, tau, r, w, max_chunk_size=30, exact=True,
                                               return_trace=True)
    res = _kernel_columns(tr, h, e, B, S, N)
    assert float(res["gate_sum"][1, 0]) == 0.0 and int(res["n_active"][1, 0]) == 0
    got = pkg.srw._diag_tuple_v401(res, N, B, S)
    assert len(got) + 1 == len(srw_ref.FUSED_V401_OUTPUT_NAMES) == 16
    for name, g, r_ in zip(srw_ref.FUSED_V401_OUTPUT_NAMES[1:], got, ref[1:]):
        g = torch.as_tensor(g, dtype=F64)
        r_ = torch.as_tensor(r_, dtype=F64)
        assert g.shape == r_.shape, name
        assert torch.allclose(g, r_, rtol=1e-6, atol=1e-9), (name, g, r_)


def test_v401_paired_16_tuple_assembly_matches_oracle(pkg):
    """The two-route form (v401:525-553): per-token outputs averaged over
    the routes, scalars over every (token, route) row."""
    B, S, D, dr, N = 2, 5, 12, 8, 72
    x, h, e, tau, r, w = _inputs(B, S, D, dr, N, seed=72)
    g = torch.Generator().manual_seed(73)
    h2 = torch.stack([h, torch.randn(B, S, dr, generator=g, dtype=F64)], dim=2)      # [B,S,2,dr]
    tau2 = torch.stack([tau, tau - 0.3], dim=2)                                       # [B,S,2,1]
    ref, tr = srw_ref.fused_gate_srw_gelu_v401_paired(x, h2, e, tau2, r, w, max_chunk_size=24,
                                                      exact=True, return_trace=True)
    T = B * S
    cols = _kernel_columns({k: (v.reshape(2 * T, *v.shape[3:]) if torch.is_tensor(v) and v.dim() == 4 else v)
                            for k, v in tr.items()}, h2.reshape(2 * T, 1, dr), e, 2 * T, 1, N)
    res = dict(token_diag=cols["token_diag"].reshape(T, 2, 14), unit_diag=cols["unit_diag"],
               gate_sum=cols["gate_sum"].reshape(T, 2), n_active=cols["n_active"].reshape(T, 2))
    got = pkg.srw._diag_tuple_v401(res, N, B, S, 2)
    for name, g_, r_ in zip(srw_ref.FUSED_V401_OUTPUT_NAMES[1:], got, ref[1:]):
        g_ = torch.as_tensor(g_, dtype=F64)
        r_ = torch.as_tensor(r_, dtype=F64)
        assert g_.shape == r_.shape, name
        assert torch.allclose(g_, r_, rtol=1e-6, atol=1e-9), (name, g_, r_)


def test_v401_factories_refuse_a_larger_mesh(pkg):
    """One GPU: a mesh with a data or model axis above 1 is refused, as for
    the v4.1 factories."""
    import pytest

    class Mesh:
        shape = {"data": 2, "model": 1}

    for make in (pkg.make_sharded_srw_v401, pkg.make_sharded_srw_paired_v401):
        with pytest.raises(NotImplementedError):
            make(Mesh())
        make(None)


def test_backward_refuses_an_unknown_gate(pkg):
    import pytest
    t = torch.zeros(4, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        pkg.srw_backward(t, t, t, torch.zeros(4, 1), t, t, t, torch.zeros(4, 1, 64), gate="relu")
