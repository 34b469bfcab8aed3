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

Prefill (more than 128 rows, d_model 256 / 512 / 1024: path
tiled_sparse_bf16): the score GEMM runs dense, then per 32-token tile the
read and write GEMMs run over the units some token of the tile passes.  The
same split holds: the sums, den, the mask and n_active equal the dense tiled
path's bit for bit (the mark kernel applies the gate kernel's arithmetic to
the same stored scores); out is within the bound above of the dense path's,
plus one more term: x.r of a listed unit is summed over eight k-slabs in LDS
instead of one MFMA chain, so bf16(x.r) may move by one ulp and P by at most
2^-6 of itself -- a further 2^-6 of sum over units of |P| |w| / den.
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


def _bound_check(inp, dense, sparse, gate, margin, den, cs, D, p_slack):
    """|sparse - dense| <= (sum over the row's non-passing units of |P| |w|) / den
    + the rounding slack: one ulp of each chunk's bf16 partial and of out, and
    p_slack (the relative change of P allowed) times sum over all units of
    |P| |w| -- not the partial's magnitude, which cancellation can make far
    smaller."""
    rows, N = gate.shape
    xb = inp["x"].to(BF)
    if rows != xb.shape[0]:                                                      # paired: x per (token, route)
        xb = xb.repeat_interleave(rows // xb.shape[0], dim=0)
    xr = srw_ref.dot_bf16(xb, inp["read"].to(BF)).float()                        # [rows, N]
    prod = srw_ref.bf16_round(srw_ref.bf16_round(gate) * xr)
    w = inp["write"].to(BF).float()                                              # [N, D]
    bound = (torch.where(margin <= 0, prod.abs(), torch.zeros(())) @ w.abs()) / den
    abs_mag = prod.abs() @ w.abs()
    chunk_mag = torch.zeros(rows, D)
    for c0 in range(0, N, cs):                                                   # the chunks' bf16 partials
        chunk_mag += srw_ref.dot_bf16(prod[:, c0:c0 + cs].to(BF), w[c0:c0 + cs].T.contiguous().to(BF)).float().abs()
    o_d = dense["out"].reshape(rows, D).float()
    o_s = sparse["out"].reshape(rows, D).float()
    slack = (chunk_mag * 2.0 ** -7 + abs_mag * p_slack) / den + o_d.abs() * 2.0 ** -7
    diff = (o_s - o_d).abs()
    print(f"  max |sparse - dense| {float(diff.max()):.3e}, max bound {float(bound.max()):.3e}", flush=True)
    assert bool((diff <= bound + slack).all())
    return o_s


TILED_CASES = [
    # T, D, dr, N, max_chunk, tau_offset, seed, routes
    (300, 1024, 1024, 3000, 1000, 1.5, 21, 1),   # configs[4]'s width; chunk ends inside union words, ragged T
    (200, 512, 128, 2600, 12500, 1.0, 22, 1),    # a router's d_route, one chunk
    (160, 256, 256, 1580, 12500, 0.8, 23, 2),    # paired routes: rows are (token, route) pairs
    (70, 1024, 1024, 700, 300, -50.0, 24, 1),    # every unit passes: the union is the pool
]
TILED_IDS = ["T{}D{}dr{}N{}c{}r{}".format(c[0], c[1], c[2], c[3], c[4], c[7]) for c in TILED_CASES]


@pytest.mark.parametrize("case", TILED_CASES, ids=TILED_IDS)
def test_tiled_sparse_within_bound_of_dense(pkg, dev, case):
    T, D, dr, N, max_chunk, tau, seed, R = case
    print(f"[gpu] tiled sparse skip {case}", flush=True)
    shape = pkg.inputs.PoolShape(T=T, D=D, N=N, dr=dr, routes=R, h_is_x=False)
    inp = pkg.inputs.make_pool_inputs(shape, seed=seed)
    inp["tau_offset"].fill_(tau)
    _, cs = srw_ref.chunk_plan(N, max_chunk)
    dense = _run(pkg, dev, inp, False, chunk_size=cs, tiled=True)
    sparse = _run(pkg, dev, inp, True, chunk_size=cs, tiled=True)
    assert dense["path"] == "tiled_bf16" and sparse["path"] == "tiled_sparse_bf16"
    for k in ("gate_sum", "den", "n_active", "pass_mask"):
        assert torch.equal(sparse[k], dense[k]), k
    rows = T * R
    if R == 1:
        ref, tr = srw_ref.fused_gate_srw(inp["x"][None], inp["h"][:, 0][None], inp["emb"], inp["tau_offset"][None],
                                         inp["read"], inp["write"], max_chunk_size=max_chunk, return_trace=True)
    else:
        ref, tr = srw_ref.fused_gate_srw_paired(inp["x"][None], inp["h"][None], inp["emb"],
                                                inp["tau_offset"].reshape(1, T, 2, 1), inp["read"], inp["write"],
                                                max_chunk_size=max_chunk, return_trace=True)
    o_s = _bound_check(inp, dense, sparse, tr["gate"].reshape(rows, N), tr["margin"].reshape(rows, N),
                       tr["den"].reshape(rows, 1), cs, D, 2.0 ** -6)
    err = rel_fro(o_s, ref[0].reshape(rows, D))
    print(f"  out rel err vs oracle {err:.3e}; active per row {sparse['n_active'].float().mean():.1f}", flush=True)
    assert err <= REL_BF16


def test_tiled_sparse_no_unit_passes(pkg, dev):
    """No unit passes anywhere: every tile's union is empty and out is zero
    (the dense path's out holds only the epsilon-sized gates' products, inside
    the bound), while the sums still count every unit."""
    T, D, dr, N = 150, 512, 512, 900
    print(f"[gpu] tiled sparse, nothing passes T{T} D{D} N{N}", flush=True)
    inp = _inputs(pkg, T, D, dr, N, 25, 4.0)
    dense = _run(pkg, dev, inp, False, tiled=True)
    sparse = _run(pkg, dev, inp, True, tiled=True)
    assert sparse["path"] == "tiled_sparse_bf16"
    for k in ("gate_sum", "den", "n_active", "pass_mask"):
        assert torch.equal(sparse[k], dense[k]), k
    assert int(sparse["n_active"].sum()) == 0
    assert not bool(sparse["out"].any())
    _, tr = srw_ref.fused_gate_srw(inp["x"][None], inp["h"][:, 0][None], inp["emb"], inp["tau_offset"][None],
                                   inp["read"], inp["write"], max_chunk_size=N, return_trace=True)
    assert int(tr["n_active"].sum()) == 0
    _bound_check(inp, dense, sparse, tr["gate"].reshape(T, N), tr["margin"].reshape(T, N),
                 tr["den"].reshape(T, 1), N, D, 2.0 ** -6)


@pytest.mark.parametrize("shape", [(300, 128, 128, 900, "mfma_ss_bf16"), (300, 1280, 128, 700, "tiled_bf16")],
                         ids=["fused", "tiled1280"])
def test_sparse_flag_runs_dense_where_no_sparse_kernel(pkg, dev, shape):
    """Shapes with no sparse kernel (more than 128 rows on the fused family,
    d_model outside 256 / 512 / 1024 on the tiled one): the flag leaves them
    on their dense matrix-core path (the same bits as without it), never on
    the scalar kernels."""
    T, D, dr, N, path = shape
    print(f"[gpu] sparse flag on a dense-only shape {shape}", flush=True)
    inp = _inputs(pkg, T, D, dr, N, 9, 0.5)
    dense = _run(pkg, dev, inp, False)
    sparse = _run(pkg, dev, inp, True)
    assert sparse["path"] == dense["path"] == path
    for k in ("out", "gate_sum", "den", "n_active", "pass_mask"):
        assert torch.equal(sparse[k], dense[k]), k
