"""GPU parity of the decode kernel (path "mfma_decode_bf16": calls of at most
128 rows, the configs[3] shape) against the CPU oracle -- fused_gate_srw
(one-pass, chunked), fused_gate_srw_paired, and _srw_inference (centred) --
with the bar of the prefill kernels (tests/test_gpu_mfma.py): out within
2e-2 relative, den and the gate sums close, the passing set identical
outside the bf16 tie band.

Shapes cover one to four 32-row blocks (T = 1, 7, 33, 100, and 64 paired =
128 rows), splits of one to four tiles, reference chunk boundaries inside a
tile, three chunks, a tail tile past N, h aliasing x, the Know pool at the
decode batch (T = 64, N = 25 200) with about half and about 3 % of the units
passing, and the Gram / centred statistics.
"""

from __future__ import annotations

import pytest
import torch

from oracle import srw_ref
from tests.parity import rel_fro, unpack_mask
from tests.test_gpu_mfma import BF, _check, _gpu, _gram_delta, _inputs, _oracle

pytestmark = pytest.mark.gpu

DECODE = "mfma_decode_bf16"

CASES = [
    # T, D, dr, N, h_is_x, max_chunk (reference), seed, tau_offset
    (64, 384, 128, 25200, False, 12500, 1, -0.5),   # Know pool, decode batch, ~50 % pass
    (64, 384, 128, 25200, False, 12500, 2, 1.38),   # ~3 % pass
    (1, 384, 128, 2600, False, 12500, 3, -0.5),     # one token
    (7, 128, 64, 777, False, 300, 4, -0.5),         # three chunks of 259 units
    (33, 384, 128, 1580, False, 12500, 5, -0.5),    # two row blocks, ragged
    (100, 128, 128, 3000, False, 1300, 6, -0.2),    # four row blocks, chunk edge inside a tile
    (50, 128, 128, 900, True, 12500, 7, -0.5),      # h aliases x
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "T{}D{}dr{}N{}{}c{}t{}".format(
    c[0], c[1], c[2], c[3], "x" if c[4] else "", c[5], c[7]))
def test_decode_matches_fused_oracle(pkg, dev, case):
    T, D, dr, N, hx, max_chunk, seed, tau = case
    print(f"[gpu] decode {case}", flush=True)
    inp = _inputs(pkg, T, D, dr, N, hx, seed, tau=tau)
    _, cs = srw_ref.chunk_plan(N, max_chunk)
    got = _gpu(pkg, dev, inp, cs)
    assert got["path"] == DECODE
    ref, tr = _oracle(inp, max_chunk)
    _check(got, ref, tr, T, N, D)


@pytest.mark.parametrize("case", [(64, 384, 128, 1580, 12500, 11), (20, 128, 64, 700, 300, 12)],
                         ids=lambda c: "T{}D{}dr{}N{}c{}".format(*c[:5]))
def test_decode_paired_matches_oracle(pkg, dev, case):
    """Paired QK routes at decode (T = 64 -> 128 rows, the configs[3] QK pool)."""
    T, D, dr, N, max_chunk, seed = case
    print(f"[gpu] decode paired {case}", flush=True)
    shape = pkg.inputs.PoolShape(T=T, D=D, N=N, dr=dr, routes=2)
    inp = pkg.inputs.make_pool_inputs(shape, seed=seed)
    _, cs = srw_ref.chunk_plan(N, max_chunk)
    got = _gpu(pkg, dev, inp, cs)
    assert got["path"] == DECODE
    ref, tr = srw_ref.fused_gate_srw_paired(
        inp["x"][None], inp["h"][None], inp["emb"], inp["tau_offset"].reshape(1, T, 2, 1),
        inp["read"], inp["write"], max_chunk_size=max_chunk, return_trace=True)
    flat = dict(margin=tr["margin"].reshape(2 * T, N), tau=tr["tau"].reshape(2 * T, 1),
                s_std=tr["s_std"].reshape(2 * T, 1), den=tr["den"].reshape(2 * T),
                gate_sum=tr["gate_sum"].reshape(2 * T), n_active=tr["n_active"].reshape(2 * T))
    got2 = {k: (v.reshape(2 * T, *v.shape[2:])[:, None] if isinstance(v, torch.Tensor) and v.dim() >= 2
                and v.shape[:2] == (T, 2) else v) for k, v in got.items()}
    _check(got2, (ref[0].reshape(2 * T, D),), flat, 2 * T, N, D)


@pytest.mark.parametrize("case", [(64, 384, 128, 25200, 21), (100, 128, 128, 3000, 22)],
                         ids=lambda c: "T{}D{}dr{}N{}".format(*c[:4]))
def test_decode_centered_matches_srw_inference_oracle(pkg, dev, case):
    """_srw_inference (v41:1713-1738) at decode: the KV-cache step's SRW layer."""
    T, D, dr, N, seed = case
    print(f"[gpu] decode centered {case}", flush=True)
    inp = _inputs(pkg, T, D, dr, N, False, seed)
    got = _gpu(pkg, dev, inp, 0, stats="centered")
    assert got["path"] == DECODE
    x = inp["x"].to(BF)
    h = inp["h"][:, 0].to(BF)
    ref, tr = srw_ref.srw_inference(x, h, inp["emb"].to(BF), inp["tau_offset"], inp["read"].to(BF),
                                    inp["write"].to(BF), return_trace=True)
    raw = tr["scores"] - tr["tau"]
    flat = dict(margin=raw - 0.5, tau=tr["tau"], s_std=tr["s_std"], den=tr["den"],
                gate_sum=tr["gate"].sum(dim=-1), n_active=(tr["activation"] > 0.5).sum(dim=-1))
    _check(got, (ref,), flat, T, N, D)


def test_decode_gram_stats_matches_oracle(pkg, dev):
    T, D, dr, N = 64, 384, 128, 25200
    print(f"[gpu] decode gram T{T} N{N}", flush=True)
    inp = _inputs(pkg, T, D, dr, N, False, 31)
    _, cs = srw_ref.chunk_plan(N, 12500)
    got = _gpu(pkg, dev, inp, cs, stats="gram")
    assert got["path"] == DECODE
    ref, tr = _oracle(inp, 12500)
    _check(got, ref, tr, T, N, D, extra_delta=_gram_delta(inp, tr))


def test_decode_rows_are_independent(pkg, dev):
    """T = 64 in one call equals the same tokens in calls of 1 and 63 rows
    (the layer is row-independent); the split geometry depends only on N, so
    each row's sums run in the same order: equal bits."""
    T, D, dr, N = 64, 384, 128, 6000
    print(f"[gpu] decode row independence T{T} N{N}", flush=True)
    inp = _inputs(pkg, T, D, dr, N, False, 41)
    inp["tau_offset"].uniform_(-0.8, 0.4, generator=torch.Generator().manual_seed(1))
    whole = _gpu(pkg, dev, inp, 0)
    parts = [_gpu(pkg, dev, dict(inp, x=inp["x"][a:b], h=inp["h"][a:b], tau_offset=inp["tau_offset"][a:b]), 0)
             for a, b in ((0, 1), (1, 64))]
    assert whole["path"] == DECODE and all(p["path"] == DECODE for p in parts)
    for k in ("out", "den", "gate_sum", "n_active", "pass_mask"):
        assert torch.equal(whole[k], torch.cat([p[k] for p in parts])), k


def test_decode_matches_prefill_kernel(pkg, dev):
    """The decode kernel and the prefill kernel on the same 128 rows: the same
    bf16 scores and gate expressions, fp32 sums in other orders."""
    T, D, dr, N = 128, 384, 128, 8000
    print(f"[gpu] decode vs prefill kernel T{T} N{N}", flush=True)
    inp = _inputs(pkg, T, D, dr, N, False, 42)
    dec = _gpu(pkg, dev, inp, 0)
    big = dict(inp, x=torch.cat([inp["x"], inp["x"]]), h=torch.cat([inp["h"], inp["h"]]),
               tau_offset=torch.cat([inp["tau_offset"], inp["tau_offset"]]))
    pre = _gpu(pkg, dev, big, 0)
    assert dec["path"] == DECODE and pre["path"] == "mfma_bf16"
    assert rel_fro(dec["out"].float(), pre["out"][:T].float()) <= 2e-3
    assert torch.allclose(dec["den"], pre["den"][:T], rtol=1e-4)
    mism = (unpack_mask(dec["pass_mask"][:, 0], N) != unpack_mask(pre["pass_mask"][:T, 0], N)).sum()
    assert int(mism) <= 4


def _pool(pkg, T, N, routes, seed, D=384, dr=128):
    shape = pkg.inputs.PoolShape(T=T, D=D, N=N, dr=dr, routes=routes)
    inp = pkg.inputs.make_pool_inputs(shape, seed=seed)
    inp["tau_offset"].uniform_(-0.9, 0.5, generator=torch.Generator().manual_seed(seed))
    return inp


def _plan(pkg, dev, inp, stats, max_chunk=12500):
    _, cs = srw_ref.chunk_plan(inp["emb"].shape[0], max_chunk)
    return pkg.SrwPlan(*(inp[k].to(BF).to(dev) if k != "tau_offset" else inp[k].to(dev)
                         for k in ("x", "h", "emb", "tau_offset", "read", "write")),
                       stats=stats, chunk_size=cs if stats == "onepass" else 0, want_mask=True)


_KEYS = ("out", "gate_sum", "den", "n_active", "pass_mask")


def _check_batch(pkg, dev, inps, stats, want_path):
    """srw_forward_batch of the calls equals their separate launches bit for
    bit: uncached, then with the pool declared cached."""
    sep = [_plan(pkg, dev, inp, stats) for inp in inps]
    for p in sep:
        p.launch()
    bat = pkg.SrwBatchPlan([_plan(pkg, dev, inp, stats) for inp in inps])
    for cached in (False, True):
        bat.launch(pool_cached=cached)
        torch.cuda.synchronize()
        assert bat.path == want_path, bat.path
        for i, (a, b) in enumerate(zip(sep, bat.plans)):
            ra, rb = a.results(), b.results()
            for k in _KEYS:
                assert torch.equal(ra[k], rb[k]), (i, k, cached)


@pytest.mark.parametrize("stats", ["onepass", "centered"])
def test_batch_qk_v_decode_one_launch_per_stage(pkg, dev, stats):
    """The QK (paired routes, 128 rows) and V calls of a decode step, as one
    launch per stage."""
    print(f"[gpu] decode batch QK+V {stats}", flush=True)
    inps = [_pool(pkg, 64, 1580, 2, 51), _pool(pkg, 64, 2600, 1, 52)]
    _check_batch(pkg, dev, inps, stats, "mfma_decode_batch_bf16")


def test_batch_three_small_pools_one_launch_per_stage(pkg, dev):
    print("[gpu] decode batch three calls", flush=True)
    inps = [_pool(pkg, 64, 1580, 1, 53), _pool(pkg, 64, 1580, 1, 54), _pool(pkg, 20, 2600, 1, 55)]
    _check_batch(pkg, dev, inps, "centered", "mfma_decode_batch_bf16")


@pytest.mark.parametrize("which", ["prefill_and_decode", "know_and_qk"])
def test_batch_that_cannot_share_launches_runs_one_by_one(pkg, dev, which):
    """A prefill-sized call with a decode-sized one, or decode calls of
    different kernel shapes (the Know pool's four-tile splits against the
    small pools' row blocks): the calls run one after the other, with the
    same results."""
    print(f"[gpu] decode batch fallback {which}", flush=True)
    if which == "prefill_and_decode":
        inps = [_pool(pkg, 300, 1580, 1, 56), _pool(pkg, 64, 2600, 1, 57)]
    else:
        inps = [_pool(pkg, 64, 25200, 1, 58), _pool(pkg, 64, 1580, 2, 59)]
    _check_batch(pkg, dev, inps, "onepass", "batch_sequential")


def test_batch_with_row_per_wave_finalize(pkg, dev):
    """Pools of under 16 splits per chunk finalize one wave per row: the
    batch takes that kernel's batch form (the model's small test pools)."""
    print("[gpu] decode batch row finalize", flush=True)
    inps = [_pool(pkg, 5, 300, 2, 60, D=128, dr=64), _pool(pkg, 5, 500, 1, 61, D=128, dr=64)]
    _check_batch(pkg, dev, inps, "centered", "mfma_decode_batch_bf16")


@pytest.mark.parametrize("dr,stats", [(384, "onepass"), (128, "onepass"), (128, "centered")])
def test_batch_prefill_qk_v_one_launch_per_stage(pkg, dev, dr, stats):
    """Prefill-sized QK (paired) and V calls of one layer (configs[1] shapes
    at 300 tokens): one launch per stage with the streaming main kernel
    (d_route = d_model) or the recomputing one (d_route = 128)."""
    print(f"[gpu] prefill batch QK+V dr{dr} {stats}", flush=True)
    inps = [_pool(pkg, 300, 1580, 2, 62, dr=dr), _pool(pkg, 300, 2600, 1, 63, dr=dr)]
    _check_batch(pkg, dev, inps, stats, "mfma_batch_bf16")
