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
