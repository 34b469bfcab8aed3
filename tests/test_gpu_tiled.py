"""GPU parity of the tiled-GEMM family ("tiled_bf16": stats, gate and write
GEMMs with the gated product P materialised as bf16) on the wide layers only
it serves -- the scaled Know pool's d_model = 1024 and the
400M / 1B models' 1280 / 2048 -- against the CPU oracle's fused_gate_srw
(models/dawn_spatial_v41_exp.py:415-635), paired routes (:640-909) and
_srw_inference (:1713-1738); and against the fused kernels where both run.

Same bar as the fused path: out within 2e-2 relative (Frobenius), den within
2e-4, the passing set identical outside a tie band of one bf16 score ulp.
"""

from __future__ import annotations

import pytest
import torch

from oracle import srw_ref
from tests.parity import gate_close, rel_fro, unpack_mask
from tests.test_gpu_mfma import _check, _gpu, _inputs, _oracle

pytestmark = pytest.mark.gpu

WIDE_CASES = [
    # T, D, dr, N, h_is_x, max_chunk, seed
    (200, 1024, 1024, 3000, True, 1000, 41),   # configs[4] widths, three reference chunks
    (130, 1280, 128, 1700, False, 12500, 42),  # 400M width with the router's d_route, ragged T/N
    (64, 2048, 2048, 700, True, 12500, 43),    # 1B width, a single partial unit tile
]


@pytest.mark.parametrize("case", WIDE_CASES, ids=lambda c: "T{}D{}dr{}N{}{}c{}".format(
    c[0], c[1], c[2], c[3], "x" if c[4] else "", c[5]))
def test_tiled_wide_matches_fused_oracle(pkg, dev, case):
    T, D, dr, N, hx, max_chunk, seed = case
    print(f"[gpu] tiled wide {case}", flush=True)
    inp = _inputs(pkg, T, D, dr, N, hx, seed)
    _, cs = srw_ref.chunk_plan(N, max_chunk)
    got = _gpu(pkg, dev, inp, cs)
    assert got["path"] == "tiled_bf16"
    ref, tr = _oracle(inp, max_chunk)
    _check(got, ref, tr, T, N, D)


def test_tiled_wide_paired(pkg, dev):
    """Paired routes at d_model = 1280: rows are (token, route) pairs, x.R^T per row."""
    T, D, dr, N = 96, 1280, 128, 1580
    print(f"[gpu] tiled wide paired T{T} D{D} N{N}", flush=True)
    shape = pkg.inputs.PoolShape(T=T, D=D, N=N, dr=dr, routes=2)
    inp = pkg.inputs.make_pool_inputs(shape, seed=44)
    got = _gpu(pkg, dev, inp, 0)
    assert got["path"] == "tiled_bf16"
    ref, tr = srw_ref.fused_gate_srw_paired(
        inp["x"][None], inp["h"][None], inp["emb"], inp["tau_offset"].reshape(1, T, 2, 1),
        inp["read"], inp["write"], max_chunk_size=12500, return_trace=True)
    flat = dict(margin=tr["margin"].reshape(2 * T, N), tau=tr["tau"].reshape(2 * T, 1),
                s_std=tr["s_std"].reshape(2 * T, 1), den=tr["den"].reshape(2 * T),
                gate_sum=tr["gate_sum"].reshape(2 * T), n_active=tr["n_active"].reshape(2 * T))
    got2 = {k: (v.reshape(2 * T, *v.shape[2:])[:, None] if isinstance(v, torch.Tensor) and v.dim() >= 2
                and v.shape[:2] == (T, 2) else v) for k, v in got.items()}
    _check(got2, (ref[0].reshape(2 * T, D),), flat, 2 * T, N, D)


def test_tiled_wide_centered(pkg, dev):
    """_srw_inference at d_model = 1024 (two-pass centred std)."""
    T, D, dr, N = 150, 1024, 1024, 2000
    print(f"[gpu] tiled wide centered T{T} N{N}", flush=True)
    inp = _inputs(pkg, T, D, dr, N, True, seed=45)
    got = _gpu(pkg, dev, inp, 0, stats="centered")
    assert got["path"] == "tiled_bf16"
    x = inp["x"].to(torch.bfloat16)
    ref, tr = srw_ref.srw_inference(x, x, inp["emb"].to(torch.bfloat16), inp["tau_offset"],
                                    inp["read"].to(torch.bfloat16), inp["write"].to(torch.bfloat16),
                                    return_trace=True)
    flat = dict(margin=tr["scores"] - tr["tau"] - 0.5, tau=tr["tau"], s_std=tr["s_std"],
                den=tr["den"], gate_sum=tr["gate"].sum(dim=-1),
                n_active=(tr["activation"] > 0.5).sum(dim=-1))
    _check(got, (ref,), flat, T, N, D)


def test_tiled_equals_fused_closely(pkg, dev):
    """Both matrix-core families on one Know-shaped input: the same bf16
    scores and gate expressions, fp32 sums in different orders."""
    T, D, dr, N = 512, 384, 384, 6000
    print(f"[gpu] tiled vs fused T{T} N{N}", flush=True)
    inp = _inputs(pkg, T, D, dr, N, True, seed=46)
    _, cs = srw_ref.chunk_plan(N, 2500)
    a = _gpu(pkg, dev, inp, cs)
    b = _gpu(pkg, dev, inp, cs, tiled=True)
    assert a["path"] in ("mfma_bf16", "mfma_ss_bf16", "mfma_decode_bf16") and b["path"] == "tiled_bf16"
    assert rel_fro(b["out"].float(), a["out"].float()) <= 2e-3
    assert torch.allclose(b["den"], a["den"], rtol=1e-4)
    mism = (unpack_mask(a["pass_mask"][:, 0], N) != unpack_mask(b["pass_mask"][:, 0], N)).sum()
    assert int(mism) <= T * N * 1e-5


def test_tiled_pool_cached(pkg, dev):
    """SRW_FLAG_POOL_CACHED reuses the packed W^T: a second call on new tokens
    with the cached pool equals a fresh call."""
    T, D, dr, N = 256, 1024, 1024, 1500
    print(f"[gpu] tiled pool cached T{T} N{N}", flush=True)
    inp = _inputs(pkg, T, D, dr, N, True, seed=47)
    bf = torch.bfloat16
    x = inp["x"].to(bf).to(dev)
    e, r, w = (inp[k].to(bf).to(dev) for k in ("emb", "read", "write"))
    tau = inp["tau_offset"].to(dev)
    plan = pkg.SrwPlan(x, x, e, tau, r, w)
    plan.launch()
    first = plan.out.clone()
    x.copy_(torch.roll(x, 1, dims=0))
    plan.launch(pool_cached=True)
    torch.cuda.synchronize()
    assert plan.path == "tiled_bf16"
    fresh = _gpu(pkg, dev, dict(inp, x=torch.roll(inp["x"], 1, dims=0)), 0)
    assert torch.equal(plan.out.cpu(), fresh["out"])
    assert torch.equal(torch.roll(first, 1, dims=0).cpu(), fresh["out"])


GATE_CASES = [
    # dtype, T, D, dr, N, stats, path
    (torch.bfloat16, 200, 128, 64, 1500, "centered", "tiled_bf16"),
    (torch.bfloat16, 130, 256, 128, 700, "onepass", "tiled_bf16"),
    (torch.float32, 150, 96, 32, 900, "centered", "tiled_f32"),
]


@pytest.mark.parametrize("case", GATE_CASES, ids=lambda c: "{}T{}D{}dr{}N{}{}".format(
    "bf16" if c[0] == torch.bfloat16 else "f32", *c[1:6]))
def test_tiled_dense_gate_output(pkg, dev, case):
    """The dense fp32 gate of every unit (_srw_inference_with_gates' gate_raw,
    v41:1741-1769) written by the tiled gate epilogue under
    SRW_FLAG_GATE_OUT: against the oracle's gates and the generic kernels'
    gates on the same inputs, with out / den unchanged from the call without
    the gate (tolerance: tests.parity.gate_close; the epilogue's exponent
    is s c + k with k = -(tau + thr) c in bf16, and its tau comes from
    one-pass sums or Chan-merged centred slices)."""
    dt, T, D, dr, N, stats, path = case
    print(f"[gpu] tiled dense gate output {case}", flush=True)
    inp = _inputs(pkg, T, D, dr, N, False, seed=46)
    x = inp["x"].to(dt).to(dev)
    h = inp["h"].to(dt).to(dev)
    args = (x, h, inp["emb"].to(dt).to(dev), inp["tau_offset"].to(dev), inp["read"].to(dt).to(dev),
            inp["write"].to(dt).to(dev))
    got = pkg.srw_forward(*args, stats=stats, want_gate=True)
    plain = pkg.srw_forward(*args, stats=stats, tiled=dt == torch.bfloat16)
    gen = pkg.srw_forward(*args, stats=stats, want_gate=True, force_generic=True)
    torch.cuda.synchronize()
    assert got["path"] == path and gen["path"] == "generic"
    assert plain["path"] == path
    for k in ("out", "den", "gate_sum", "n_active"):
        assert torch.equal(got[k].cpu(), plain[k].cpu()), k
    g = got["gate"].cpu().reshape(T, N)
    h1, e1 = inp["h"][:, 0].to(dt), inp["emb"].to(dt)
    ok, n = gate_close(g, gen["gate"].cpu().reshape(T, N), h1, e1)
    print(f"  compared {n} of {T * N} gates (tie band excluded)", flush=True)
    assert ok
    if stats == "centered":
        _, rg, _ = srw_ref.srw_inference_with_gates(inp["x"].to(dt), h1, e1, inp["tau_offset"], inp["read"].to(dt),
                                                    inp["write"].to(dt))
        assert gate_close(g, rg.reshape(T, N), h1, e1)[0]
    # the gate sums of the dense gate are the call's gate_sum
    assert torch.allclose(g.sum(dim=-1), got["gate_sum"].cpu().reshape(T), rtol=1e-4, atol=1e-6)
