"""GPU parity: libsrw_amd.so (through its C ABI) vs the CPU oracle.

Every test prints the case it runs before touching the GPU.
"""

from __future__ import annotations

import pytest
import torch

from oracle import srw_ref
from tests.parity import (REL_BF16, REL_F32, ROW_REL_BF16, assert_pass_set, bf16_ulp, gate_close,
                          rel_fro, row_rel_max, unpack_mask)

pytestmark = pytest.mark.gpu

BF = torch.bfloat16
F32 = torch.float32


def _inputs(pkg, T, D, dr, N, R=1, h_is_x=False, seed=0, tau=-0.5):
    shape = pkg.inputs.PoolShape(T=T, D=D, N=N, dr=dr, routes=R, h_is_x=h_is_x)
    inp = pkg.inputs.make_pool_inputs(shape, seed=seed)
    if tau is not None:
        inp["tau_offset"].fill_(tau)
    return inp


def _run(pkg, inp, dev, dtype, **kw):
    x = inp["x"].to(dtype).to(dev)
    h = x if "h" not in inp else inp["h"].to(dtype).to(dev)
    res = pkg.srw_forward(x, h, inp["emb"].to(dtype).to(dev), inp["tau_offset"].to(dev),
                          inp["read"].to(dtype).to(dev), inp["write"].to(dtype).to(dev), **kw)
    torch.cuda.synchronize()
    return {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in res.items()}


def _oracle_fused(inp, chunk, routes):
    x = inp["x"][None]
    T = x.shape[1]
    if routes == 1:
        h = x if "h" not in inp else inp["h"][:, 0][None]
        tau = inp["tau_offset"][None]
        return srw_ref.fused_gate_srw(x, h, inp["emb"], tau, inp["read"], inp["write"],
                                      max_chunk_size=chunk, return_trace=True)
    h = inp["h"][None]
    tau = inp["tau_offset"].reshape(1, T, routes, 1)
    return srw_ref.fused_gate_srw_paired(x, h, inp["emb"], tau, inp["read"], inp["write"],
                                         max_chunk_size=chunk, return_trace=True)


BF16_CASES = [
    # T, D, dr, N, R, h_is_x, max_chunk
    (1, 64, 64, 64, 1, True, 2048),
    (5, 64, 32, 100, 1, False, 2048),
    (33, 128, 64, 1000, 1, False, 300),
    (64, 384, 384, 2600, 1, True, 2048),
    (40, 384, 128, 1580, 2, False, 2048),
    (7, 40, 24, 77, 1, False, 10),
    (16, 1024, 1024, 3000, 1, True, 1000),
]


@pytest.mark.parametrize("case", BF16_CASES, ids=lambda c: "T{}D{}dr{}N{}R{}{}c{}".format(
    c[0], c[1], c[2], c[3], c[4], "x" if c[5] else "", c[6]))
def test_generic_bf16_emulation_matches_fused_oracle(pkg, dev, case):
    T, D, dr, N, R, hx, chunk = case
    print(f"[gpu] generic bf16 emulate {case}", flush=True)
    inp = _inputs(pkg, T, D, dr, N, R, hx, seed=T + N)
    nc, cs = srw_ref.chunk_plan(N, chunk)
    got = _run(pkg, inp, dev, BF, stats="onepass", chunk_size=cs, emulate=True, diag=True)
    assert got["path"] == "generic"
    ref, tr = _oracle_fused(inp, chunk, R)
    out_ref = ref[0].reshape(T, R, D)
    out = got["out"].float()
    assert rel_fro(out, out_ref) <= 2e-3
    assert row_rel_max(out, out_ref) <= 2e-2
    den_ref = tr["den"].reshape(T, R)
    assert torch.allclose(got["den"], den_ref, rtol=1e-4, atol=0)
    assert torch.allclose(got["gate_sum"], tr["gate_sum"].reshape(T, R), rtol=1e-3, atol=1e-6)
    # passing set inside the tie band (bf16: one score ulp + tau slack)
    margin = tr["margin"].reshape(T, R, N)
    score = margin + tr["tau"].reshape(T, R, 1) + 0.5
    delta = bf16_ulp(score) + 1e-4 * tr["s_std"].reshape(T, R, 1)
    mask = unpack_mask(got["pass_mask"], N)
    n_mis = assert_pass_set(mask, margin, delta)
    na_ref = tr["n_active"].reshape(T, R)
    assert (got["n_active"].float() - na_ref).abs().max() <= max(2, n_mis)


F32_CASES = [
    (1, 64, 64, 64, True),
    (9, 96, 48, 333, False),
    (32, 384, 384, 2600, True),
    (16, 384, 128, 5000, False),
]


@pytest.mark.parametrize("case", F32_CASES, ids=lambda c: "T{}D{}dr{}N{}{}".format(
    c[0], c[1], c[2], c[3], "x" if c[4] else ""))
def test_generic_f32_matches_srw_inference(pkg, dev, case):
    T, D, dr, N, hx = case
    print(f"[gpu] generic f32 centered {case}", flush=True)
    inp = _inputs(pkg, T, D, dr, N, 1, hx, seed=3 * T + N)
    got = _run(pkg, inp, dev, F32, stats="centered", want_mask=True, force_generic=True)
    assert got["path"] == "generic"
    h = inp["x"] if hx else inp["h"][:, 0]
    out_ref, tr = srw_ref.srw_inference(inp["x"], h, inp["emb"], inp["tau_offset"],
                                        inp["read"], inp["write"], return_trace=True)
    assert rel_fro(got["out"][:, 0], out_ref) <= REL_F32
    margin = tr["margin"]
    delta = 1e-5 * torch.clamp_min(tr["s_std"], 1.0)
    assert_pass_set(unpack_mask(got["pass_mask"], N)[:, 0], margin, delta)


def test_generic_gelu_v401_f32(pkg, dev):
    T, D, dr, N = 24, 128, 64, 900
    print(f"[gpu] generic gelu v401 f32 T{T} D{D} dr{dr} N{N}", flush=True)
    inp = _inputs(pkg, T, D, dr, N, seed=11)
    inp["tau_offset"].fill_(0.7)
    got = _run(pkg, inp, dev, F32, gate="gelu_v401", stats="centered", force_generic=True)
    assert got["path"] == "generic"
    ref = srw_ref.srw_inference_gelu_v401(inp["x"], inp["h"][:, 0], inp["emb"], inp["tau_offset"],
                                          inp["read"], inp["write"])
    assert rel_fro(got["out"][:, 0], ref) <= REL_F32


def test_generic_gelu_v401_bf16_fused(pkg, dev):
    T, D, dr, N = 24, 128, 64, 900
    print(f"[gpu] generic gelu v401 bf16 T{T} D{D} dr{dr} N{N}", flush=True)
    inp = _inputs(pkg, T, D, dr, N, seed=12)
    inp["tau_offset"].fill_(0.3)
    nc, cs = srw_ref.chunk_plan(N, 400)
    got = _run(pkg, inp, dev, BF, gate="gelu_v401", stats="onepass", chunk_size=cs, emulate=True)
    ref = srw_ref.fused_gate_srw_gelu_v401(inp["x"][None], inp["h"][:, 0][None], inp["emb"],
                                           inp["tau_offset"][None], inp["read"], inp["write"],
                                           max_chunk_size=400)
    assert rel_fro(got["out"][:, 0].float(), ref[0][0]) <= 5e-3


def test_dropin_fused_single_22_tuple(pkg, dev):
    B, S, D, dr, N = 2, 24, 128, 64, 1200
    print(f"[gpu] drop-in make_sharded_srw B{B} S{S} D{D} dr{dr} N{N}", flush=True)
    inp = _inputs(pkg, B * S, D, dr, N, seed=5)
    x = inp["x"].reshape(B, S, D)
    h = inp["h"].reshape(B, S, dr)
    tau = inp["tau_offset"].reshape(B, S, 1)
    fn = pkg.make_sharded_srw(None, max_chunk_size=500)
    got = fn(x.to(dev), h.to(dev), inp["emb"].to(dev), tau.to(dev), inp["read"].to(dev),
             inp["write"].to(dev))
    torch.cuda.synchronize()
    ref = srw_ref.fused_gate_srw(x, h, inp["emb"], tau, inp["read"], inp["write"],
                                 max_chunk_size=500)
    assert len(got) == 22
    assert rel_fro(got[0].cpu(), ref[0]) <= REL_BF16
    for i, name in enumerate(srw_ref.FUSED_OUTPUT_NAMES[1:], start=1):
        g, r = got[i].detach().cpu().float(), ref[i].float()
        assert g.shape == r.shape, name
        assert torch.allclose(g, r, rtol=2e-2, atol=2e-3), (name, g, r)


def test_dropin_fused_paired_22_tuple(pkg, dev):
    B, S, D, dr, N = 2, 16, 128, 64, 700
    print(f"[gpu] drop-in make_sharded_srw_paired B{B} S{S} D{D} dr{dr} N{N}", flush=True)
    inp = _inputs(pkg, B * S, D, dr, N, R=2, seed=6)
    x = inp["x"].reshape(B, S, D)
    h = inp["h"].reshape(B, S, 2, dr)
    tau = inp["tau_offset"].reshape(B, S, 2, 1)
    fn = pkg.make_sharded_srw_paired(None, max_chunk_size=2048)
    got = fn(x.to(dev), h.to(dev), inp["emb"].to(dev), tau.to(dev), inp["read"].to(dev),
             inp["write"].to(dev))
    torch.cuda.synchronize()
    ref = srw_ref.fused_gate_srw_paired(x, h, inp["emb"], tau, inp["read"], inp["write"],
                                        max_chunk_size=2048)
    assert got[0].shape == (B, S, 2, D)
    assert rel_fro(got[0].cpu(), ref[0]) <= REL_BF16
    for i, name in enumerate(srw_ref.FUSED_OUTPUT_NAMES[1:], start=1):
        g, r = got[i].detach().cpu().float(), ref[i].float()
        assert g.shape == r.shape, name
        assert torch.allclose(g, r, rtol=2e-2, atol=2e-3), (name, g, r)


def test_dropin_srw_inference_f32(pkg, dev):
    B, S, D, dr, N = 2, 8, 96, 32, 500
    print(f"[gpu] drop-in srw_inference f32 B{B} S{S}", flush=True)
    inp = _inputs(pkg, B * S, D, dr, N, seed=8)
    x = inp["x"].reshape(B, S, D)
    h = inp["h"].reshape(B, S, dr)
    tau = inp["tau_offset"].reshape(B, S, 1)
    got = pkg.srw_inference(x.to(dev), h.to(dev), inp["emb"].to(dev), tau.to(dev),
                            inp["read"].to(dev), inp["write"].to(dev))
    ref = srw_ref.srw_inference(x, h, inp["emb"], tau, inp["read"], inp["write"])
    assert got.dtype == F32 and got.shape == (B, S, D)
    assert rel_fro(got.cpu(), ref) <= REL_F32


def test_den_floor_small_pool(pkg, dev):
    """QK/V-sized pools with a high tau_offset: den = max(sum intensity, 1) floors at 1."""
    T, D, dr, N = 16, 128, 64, 1580
    print(f"[gpu] den floor T{T} N{N}", flush=True)
    inp = _inputs(pkg, T, D, dr, N, seed=21, tau=3.0)
    nc, cs = srw_ref.chunk_plan(N, 2048)
    got = _run(pkg, inp, dev, BF, stats="onepass", chunk_size=cs, emulate=True)
    ref, tr = _oracle_fused(inp, 2048, 1)
    assert (tr["intensity_sum"] < 1).any()
    assert torch.equal(got["den"][:, 0] == 1.0, tr["den"].reshape(T) == 1.0)
    assert rel_fro(got["out"][:, 0].float(), ref[0][0]) <= 2e-3


def test_empty_tokens(pkg, dev):
    print("[gpu] T=0", flush=True)
    x = torch.empty(0, 64, dtype=BF, device=dev)
    h = torch.empty(0, 1, 32, dtype=BF, device=dev)
    e = torch.randn(10, 32, device=dev).to(BF)
    rw = torch.randn(10, 64, device=dev).to(BF)
    tau = torch.empty(0, 1, device=dev)
    res = pkg.srw_forward(x, h, e, tau, rw, rw)
    assert res["out"].shape == (0, 1, 64) and res["path"] == "empty"


@pytest.mark.parametrize("dtype", [F32, BF])
def test_dropin_srw_inference_with_gates(pkg, dev, dtype):
    """_srw_inference_with_gates (v41:1741-1769): out, the dense gate of every
    unit and its row-normalised form, against the oracle."""
    B, S, D, dr, N = 2, 12, 96, 32, 700
    print(f"[gpu] drop-in srw_inference_with_gates {dtype} B{B} S{S} N{N}", flush=True)
    inp = _inputs(pkg, B * S, D, dr, N, seed=9)
    x = inp["x"].reshape(B, S, D).to(dtype)
    h = inp["h"].reshape(B, S, dr).to(dtype)
    tau = inp["tau_offset"].reshape(B, S, 1)
    emb, rd, wr = (inp[k].to(dtype) for k in ("emb", "read", "write"))
    out, g, gn = pkg.srw_inference_with_gates(x.to(dev), h.to(dev), emb.to(dev), tau.to(dev),
                                              rd.to(dev), wr.to(dev))
    ro, rg, rgn = srw_ref.srw_inference_with_gates(x, h, emb, tau, rd, wr)
    assert out.dtype == F32 and out.shape == (B, S, D)
    assert g.shape == (B, S, N) and gn.shape == (B, S, N)
    tol = REL_F32 if dtype == F32 else REL_BF16
    assert rel_fro(out.cpu(), ro) <= tol
    # the gate itself is fp32 in both dtypes (scores are rounded to the input
    # dtype first); tolerance and tie band: tests.parity.gate_close
    assert gate_close(g.cpu().reshape(B * S, N), rg.reshape(B * S, N), h.reshape(B * S, dr), emb)[0]
    assert gate_close(gn.cpu().reshape(B * S, N), rgn.reshape(B * S, N), h.reshape(B * S, dr), emb)[0]
    assert torch.allclose(gn.sum(dim=-1).cpu(), torch.ones(B, S), atol=1e-4)
