"""GPU: the sparse-skip decode kernel (SRW_FLAG_SPARSE_SKIP, calls of at most
128 rows) against the dense decode kernel and the oracle.

The sparse kernel reads the R row of a unit and the W^T fragment halves of
an 8-unit group only when some row of the workgroup passes there (north
star: unit rows whose gate is zero across the tile are skipped).

* v4.0.1 GELU gate: a unit that no row passes has gate 0 for every row
  (v401:305-306), so skipping it changes nothing -- every output is
  bit-identical to the dense kernel's.
* v4.1 gate: such a unit's gate is the epsilon-sized sigmoid(500 margin)
  (intensity) < 0.5 epsilon (v41:505-511), which the dense kernel folds into
  out.  The gate and intensity sums, den, the pass mask and n_active are
  still computed from every unit's score and are bit-identical; out differs
  from the dense kernel's by at most sum over the token's non-passing units
  |bf16(bf16(gate) x.r)| |w| / den (each skipped unit is non-passing for the
  token), evaluated from the oracle's gates, plus the rounding slack: each
  reference chunk's partial write GEMM is rounded to bf16 before the chunks
  are summed (v41:518), so a change below the bound can move a chunk's
  rounding by one ulp (<= 2^-7 of its magnitude), and out by one ulp more.
"""

from __future__ import annotations

import pytest
import torch

from oracle import srw_ref
from tests.parity import REL_BF16, rel_fro

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


def _inputs(pkg, T, D, dr, N, seed, tau):
    shape = pkg.inputs.PoolShape(T=T, D=D, N=N, dr=dr, routes=1, h_is_x=False)
    inp = pkg.inputs.make_pool_inputs(shape, seed=seed)
    inp["tau_offset"].fill_(tau)
    return inp


def _run(pkg, dev, inp, sparse, **kw):
    x = inp["x"].to(BF).to(dev)
    h = inp["h"].to(BF).to(dev)
    res = pkg.srw_forward(x, h, inp["emb"].to(BF).to(dev), inp["tau_offset"].to(dev),
                          inp["read"].to(BF).to(dev), inp["write"].to(BF).to(dev),
                          sparse_skip=sparse, want_mask=True, **kw)
    torch.cuda.synchronize()
    return {k: (v.cpu() if isinstance(v, torch.Tensor) else v) for k, v in res.items()}


CASES = [
    # T, D, dr, N, max_chunk, tau_offset, seed: tau high -> few units pass
    (1, 384, 128, 25200, 12600, 2.0, 1),    # one token, the Know pool
    (8, 384, 128, 25200, 12600, 2.0, 2),
    (64, 384, 128, 25200, 12600, 2.0, 3),   # configs[3]'s batch of 64
    (40, 128, 64, 2600, 1300, 1.5, 4),      # ragged T, chunk boundary
    (100, 128, 128, 777, 300, 0.5, 5),      # four row blocks, three chunks
]
IDS = ["T{}D{}dr{}N{}".format(*c[:4]) for c in CASES]


@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_sparse_skip_gelu_equals_dense(pkg, dev, case):
    T, D, dr, N, max_chunk, tau, seed = case
    print(f"[gpu] sparse-skip gelu v401 {case}", flush=True)
    inp = _inputs(pkg, T, D, dr, N, seed, tau)
    _, cs = srw_ref.chunk_plan(N, max_chunk)
    dense = _run(pkg, dev, inp, False, gate="gelu_v401", chunk_size=cs)
    sparse = _run(pkg, dev, inp, True, gate="gelu_v401", chunk_size=cs)
    assert dense["path"] == "mfma_decode_bf16" and sparse["path"] == "mfma_decode_sparse_bf16"
    for k in ("out", "gate_sum", "den", "n_active", "pass_mask"):
        assert torch.equal(sparse[k], dense[k]), k
    x = inp["x"][None]
    ref = srw_ref.fused_gate_srw_gelu_v401(x, inp["h"][:, 0][None], inp["emb"], inp["tau_offset"][None],
                                           inp["read"], inp["write"], max_chunk_size=max_chunk)
    err = rel_fro(sparse["out"][:, 0].float(), ref[0][0])
    print(f"  out rel err vs oracle {err:.3e}; active per row {sparse['n_active'].float().mean():.1f}", flush=True)
    assert err <= REL_BF16


@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_sparse_skip_v41_within_bound_of_dense(pkg, dev, case):
    T, D, dr, N, max_chunk, tau, seed = case
    print(f"[gpu] sparse-skip v4.1 {case}", flush=True)
    inp = _inputs(pkg, T, D, dr, N, seed, tau)
    _, cs = srw_ref.chunk_plan(N, max_chunk)
    dense = _run(pkg, dev, inp, False, chunk_size=cs)
    sparse = _run(pkg, dev, inp, True, chunk_size=cs)
    assert dense["path"] == "mfma_decode_bf16" and sparse["path"] == "mfma_decode_sparse_bf16"
    for k in ("gate_sum", "den", "n_active", "pass_mask"):
        assert torch.equal(sparse[k], dense[k]), k
    # the bound: every skipped unit is non-passing for the token
    x = inp["x"][None]
    ref, tr = srw_ref.fused_gate_srw(x, inp["h"][:, 0][None], inp["emb"], inp["tau_offset"][None],
                                     inp["read"], inp["write"], max_chunk_size=max_chunk, return_trace=True)
    gate = tr["gate"].reshape(T, N)
    margin = tr["margin"].reshape(T, N)
    den = tr["den"].reshape(T, 1)
    xr = srw_ref.dot_bf16(inp["x"].to(BF), inp["read"].to(BF)).float()          # [T, N]
    prod = srw_ref.bf16_round(srw_ref.bf16_round(gate) * xr)
    w = inp["write"].to(BF).float()                                              # [N, D]
    p_skip = torch.where(margin <= 0, prod.abs(), torch.zeros(()))
    bound = (p_skip @ w.abs()) / den
    chunk_mag = torch.zeros(T, D)
    for c0 in range(0, N, cs):                                                   # the chunks' bf16 partials
        chunk_mag += srw_ref.dot_bf16(prod[:, c0:c0 + cs].to(BF), w[c0:c0 + cs].T.contiguous().to(BF)).float().abs()
    o_d, o_s = dense["out"][:, 0].float(), sparse["out"][:, 0].float()
    slack = chunk_mag * 2.0 ** -7 / den + o_d.abs() * 2.0 ** -7
    diff = (o_s - o_d).abs()
    print(f"  max |sparse - dense| {float(diff.max()):.3e}, max bound {float(bound.max()):.3e}", flush=True)
    assert bool((diff <= bound + slack).all())
    err = rel_fro(o_s, ref[0].reshape(T, D))
    print(f"  out rel err vs oracle {err:.3e}", flush=True)
    assert err <= REL_BF16


@pytest.mark.parametrize("shape", [(300, 128, 128, 900, "mfma_ss_bf16"), (300, 1024, 1024, 700, "tiled_bf16")],
                         ids=["fused", "tiled"])
def test_sparse_flag_runs_dense_where_no_sparse_kernel(pkg, dev, shape):
    """Prefill shapes have no sparse kernel: the flag leaves them on their
    dense matrix-core path (the same bits as without it), never on the
    scalar kernels."""
    T, D, dr, N, path = shape
    print(f"[gpu] sparse flag on a prefill shape {shape}", flush=True)
    inp = _inputs(pkg, T, D, dr, N, 9, 0.5)
    dense = _run(pkg, dev, inp, False)
    sparse = _run(pkg, dev, inp, True)
    assert sparse["path"] == dense["path"] == path
    for k in ("out", "gate_sum", "den", "n_active", "pass_mask"):
        assert torch.equal(sparse[k], dense[k]), k
