"""GPU parity of the fp32 matrix-core family (``tiled_f32``:
srw_tiled_f32.hip, v_mfma_f32_32x32x2_f32) through the C ABI.

* Centred statistics (the fp32 ``_srw_inference``, v41:1713-1738) against
  the oracle's ``srw_inference`` (pinned on the CPU, tests/test_oracle_pins.py):
  out within 1e-5 relative (Frobenius), den within 1e-5, the passing set
  identical outside a band of 1e-5 max(s_std, 1) around the threshold (fp32
  scores summed in another order).
* One-pass statistics in fp32 (fused_gate_srw's moments, v41:434-462, on
  fp32 inputs): against the reference-faithful scalar kernels (the generic
  family, pinned to the oracle in tests/test_gpu_parity.py) to the same bar.
* configs[0] as written: the full T = 4096 x N = 25 200 Know-pool call in
  fp32, 512 of its rows against the oracle (rows are independent).
* The v4.0.1 ``_srw_inference`` in fp32 (v401:1443-1463: forward-normalised
  rows, z Phi(z) gate, den = max(sum gate, 1)) against the oracle's
  ``srw_inference_gelu_v401``, to the same bar (pass <=> z > 0).
"""

from __future__ import annotations

import pytest
import torch

from oracle import srw_ref
from tests.parity import REL_F32, assert_pass_set, rel_fro, unpack_mask

pytestmark = pytest.mark.gpu

F32 = torch.float32


def _inputs(pkg, T, D, dr, N, R, h_is_x, seed, tau):
    shape = pkg.inputs.PoolShape(T=T, D=D, N=N, dr=dr, routes=R, h_is_x=h_is_x)
    inp = pkg.inputs.make_pool_inputs(shape, seed=seed)
    inp["tau_offset"].uniform_(tau - 0.3, tau + 0.3, generator=torch.Generator().manual_seed(seed))
    return inp


def _gpu(pkg, dev, inp, **kw):
    x = inp["x"].to(dev)
    h = x if "h" not in inp else inp["h"].to(dev)
    res = pkg.srw_forward(x, h, inp["emb"].to(dev), inp["tau_offset"].to(dev), inp["read"].to(dev),
                          inp["write"].to(dev), want_mask=True, **kw)
    torch.cuda.synchronize()
    return {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in res.items()}


CENTRED = [
    # T, D, dr, N, R, h_is_x, tau_offset, seed
    (1, 64, 64, 64, 1, True, -0.5, 1),          # one row, one partial tile
    (32, 384, 384, 2600, 1, True, 0.3, 2),      # h aliases x
    (300, 384, 128, 5000, 1, False, 0.8, 3),    # two token tiles, ragged
    (77, 128, 64, 777, 2, False, 0.0, 4),       # paired routes: 154 virtual rows
    (40, 256, 96, 300, 1, False, 1.5, 5),       # few units pass; N below one tile
    (70, 1152, 64, 1000, 1, False, 0.4, 8),     # three 384-wide write column tiles
]


@pytest.mark.parametrize("case", CENTRED, ids=lambda c: "T{}D{}dr{}N{}R{}{}".format(
    c[0], c[1], c[2], c[3], c[4], "x" if c[5] else ""))
def test_f32_centred_matches_srw_inference(pkg, dev, case):
    T, D, dr, N, R, hx, tau, seed = case
    print(f"[gpu] tiled f32 centred {case}", flush=True)
    inp = _inputs(pkg, T, D, dr, N, R, hx, seed, tau)
    got = _gpu(pkg, dev, inp, stats="centered")
    assert got["path"] == "tiled_f32"
    for r in range(R):
        h = inp["x"] if hx else inp["h"][:, r]
        ref, tr = srw_ref.srw_inference(inp["x"], h, inp["emb"], inp["tau_offset"][:, r:r + 1], inp["read"],
                                        inp["write"], return_trace=True)
        err = rel_fro(got["out"][:, r], ref)
        print(f"  route {r}: out rel err {err:.3e}", flush=True)
        assert got["out"].dtype == F32
        assert err <= REL_F32
        assert torch.allclose(got["den"][:, r], tr["den"][:, 0], rtol=1e-5)
        delta = 1e-5 * torch.clamp_min(tr["s_std"], 1.0)
        mask = unpack_mask(got["pass_mask"][:, r], N)
        assert_pass_set(mask, tr["margin"], delta)
        assert torch.equal(got["n_active"][:, r].long(), mask.sum(dim=1))


@pytest.mark.parametrize("case", [(200, 384, 128, 1580, 1, False, 0.5, 6), (64, 128, 128, 900, 2, False, 0.2, 7)],
                         ids=["R1", "R2"])
def test_f32_onepass_matches_generic(pkg, dev, case):
    T, D, dr, N, R, hx, tau, seed = case
    print(f"[gpu] tiled f32 one-pass vs generic {case}", flush=True)
    inp = _inputs(pkg, T, D, dr, N, R, hx, seed, tau)
    got = _gpu(pkg, dev, inp, stats="onepass")
    gen = _gpu(pkg, dev, inp, stats="onepass", force_generic=True)
    assert got["path"] == "tiled_f32" and gen["path"] == "generic"
    err = rel_fro(got["out"], gen["out"])
    print(f"  out rel err vs generic {err:.3e}", flush=True)
    assert err <= REL_F32
    assert torch.allclose(got["den"], gen["den"], rtol=1e-5)
    assert torch.allclose(got["gate_sum"], gen["gate_sum"], rtol=1e-4, atol=1e-6)
    mism = (unpack_mask(got["pass_mask"], N) != unpack_mask(gen["pass_mask"], N)).sum()
    assert int(mism) <= 2


def test_configs0_fp32_full_call(pkg, dev):
    """configs[0] as written: fp32 _srw_inference of the whole T = 4096 batch
    over the full Know pool on the matrix cores; rows 0..255 and the last 256
    against the oracle."""
    shape = pkg.inputs.CONFIGS["know"]
    print(f"[gpu] configs[0] fp32 full call T{shape.T} D{shape.D} N{shape.N}", flush=True)
    inp = pkg.inputs.make_pool_inputs(shape, seed=0)
    x = inp["x"].to(dev)
    res = pkg.srw_forward(x, x, inp["emb"].to(dev), inp["tau_offset"].to(dev), inp["read"].to(dev),
                          inp["write"].to(dev), stats="centered", want_mask=True)
    torch.cuda.synchronize()
    assert res["path"] == "tiled_f32"
    out = res["out"][:, 0].cpu()
    assert bool(torch.isfinite(out).all())
    rows = torch.cat([torch.arange(256), torch.arange(shape.T - 256, shape.T)])
    xs = inp["x"][rows]
    ref, tr = srw_ref.srw_inference(xs, xs, inp["emb"], inp["tau_offset"][rows], inp["read"], inp["write"],
                                    return_trace=True)
    err = rel_fro(out[rows], ref)
    print(f"  out rel err on {len(rows)} rows {err:.3e}", flush=True)
    assert err <= REL_F32
    assert torch.allclose(res["den"][rows, 0].cpu(), tr["den"][:, 0], rtol=1e-5)
    delta = 1e-5 * torch.clamp_min(tr["s_std"], 1.0)
    assert_pass_set(unpack_mask(res["pass_mask"][rows, 0].cpu(), shape.N), tr["margin"], delta)


V401 = [
    # T, D, dr, N, R, h_is_x, tau_offset, seed
    (150, 384, 128, 2600, 1, False, 0.6, 11),   # the reference's inference shape family, ragged
    (64, 96, 32, 700, 1, False, 1.2, 12),       # narrow widths, a partial unit tile
    (40, 128, 128, 900, 2, False, 0.3, 13),     # paired routes
]


@pytest.mark.parametrize("case", V401, ids=lambda c: "T{}D{}dr{}N{}R{}".format(*c[:5]))
def test_f32_gelu_v401_matches_srw_inference(pkg, dev, case):
    T, D, dr, N, R, hx, tau, seed = case
    print(f"[gpu] tiled f32 v4.0.1 srw_inference {case}", flush=True)
    inp = _inputs(pkg, T, D, dr, N, R, hx, seed, tau)
    got = _gpu(pkg, dev, inp, stats="centered", gate="gelu_v401")
    assert got["path"] == "tiled_f32"
    for r in range(R):
        h = inp["h"][:, r]
        ref, tr = srw_ref.srw_inference_gelu_v401(inp["x"], h, inp["emb"], inp["tau_offset"][:, r:r + 1],
                                                  inp["read"], inp["write"], return_trace=True)
        err = rel_fro(got["out"][:, r], ref)
        print(f"  route {r}: out rel err {err:.3e}, active per row {got['n_active'][:, r].float().mean():.1f}",
              flush=True)
        assert err <= REL_F32
        assert torch.allclose(got["den"][:, r], tr["den"][:, 0], rtol=1e-5)
        assert torch.allclose(got["gate_sum"][:, r], tr["gate"].sum(dim=-1), rtol=1e-5, atol=1e-6)
        # pass <=> z > 0 <=> s - tau > 0, band as for the v4.1 margin
        raw = tr["z"] * tr["s_std"]
        delta = 1e-5 * torch.clamp_min(tr["s_std"], 1.0)
        mask = unpack_mask(got["pass_mask"][:, r], N)
        assert_pass_set(mask, raw, delta)
        assert torch.equal(got["n_active"][:, r].long(), mask.sum(dim=1))

