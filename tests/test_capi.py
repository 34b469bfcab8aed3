"""CPU checks of the C ABI: the library loads, exports every symbol the
header declares, its struct layouts match the ctypes mirror (checked with a
gcc-compiled probe of include/srw_amd.h), and argument validation returns
the documented status codes without touching a GPU."""

from __future__ import annotations

import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "srw_amd.h")


@pytest.fixture(scope="module")
def C(pkg):
    from dawn_srw_amd import _capi
    _capi.load_library()
    return _capi


def _header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"^\s*[A-Za-z_][\w\s\*]*?\b(srw_\w+)\s*\(", text, flags=re.M))


def test_library_exports_every_header_symbol(C):
    declared = _header_functions()
    assert declared == set(C.EXPORTED_SYMBOLS)
    lib = C.load_library()
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.srw_abi_version() == C.ABI_VERSION


def test_struct_layout_matches_header(C, tmp_path):
    fields = [f[0] for f in C.SrwDesc._fields_]
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "srw_amd.h"', "int main(void){",
             'printf("%zu %zu %zu %zu %zu %d %d\\n", sizeof(srw_desc_t), sizeof(srw_tensors_t), '
             'sizeof(srw_outputs_t), sizeof(srw_cotangents_t), sizeof(srw_grads_t), '
             '(int)SRW_TDIAG_COUNT, (int)SRW_UDIAG_COUNT);']
    for f in fields:
        lines.append(f'printf("{f} %zu\\n", offsetof(srw_desc_t, {f}));')
    lines.append("return 0;}")
    src = tmp_path / "probe.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "probe"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", os.path.dirname(HEADER),
                    str(src), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    sizes = [int(v) for v in out[0].split()]
    assert sizes == [ctypes.sizeof(C.SrwDesc), ctypes.sizeof(C.SrwTensors),
                     ctypes.sizeof(C.SrwOutputs), ctypes.sizeof(C.SrwCotangents),
                     ctypes.sizeof(C.SrwGrads), len(C.TDIAG), len(C.UDIAG)]
    for line in out[1:]:
        if line:
            name, off = line.split()
            assert getattr(C.SrwDesc, name).offset == int(off), name


def test_desc_init_reference_defaults(C):
    d = C.desc_init()
    # models/dawn_spatial_v41_exp.py:297-301, :352
    assert (d.sharpness, d.act_threshold, d.epsilon, d.max_intensity) == (500.0, 0.5,
                                                                           ctypes.c_float(1e-4).value, 10.0)
    assert d.act_cutoff == ctypes.c_float(0.01).value
    assert d.dead_threshold == ctypes.c_float(0.01).value
    assert (d.n_routes, d.dtype, d.gate, d.stats_mode, d.scale) == (1, C.SRW_BF16, C.SRW_GATE_V41,
                                                                    C.SRW_STATS_ONEPASS, 1.0)


def _desc(C, **kw):
    d = C.desc_init()
    d.T, d.d_model, d.d_route, d.n_units = 16, 64, 32, 100
    for k, v in kw.items():
        setattr(d, k, v)
    return d


@pytest.mark.parametrize("bad", [dict(T=-1), dict(d_model=0), dict(n_units=0), dict(n_routes=3),
                                 dict(dtype=7), dict(gate=9), dict(stats_mode=5),
                                 dict(chunk_size=-2), dict(flags=0x100),
                                 dict(sharpness=float("nan"))])
def test_invalid_descriptors_rejected(C, bad):
    d = _desc(C, **bad)
    n = ctypes.c_size_t(0)
    assert C.load_library().srw_workspace_size(ctypes.byref(d), ctypes.byref(n)) == C.SRW_EINVAL
    t, o = C.SrwTensors(), C.SrwOutputs()
    st = C.load_library().srw_forward(ctypes.byref(d), ctypes.byref(t), ctypes.byref(o), None, 0, None)
    assert st == C.SRW_EINVAL


def test_null_pointers_rejected_before_any_launch(C):
    d = _desc(C)
    t, o = C.SrwTensors(), C.SrwOutputs()
    st = C.load_library().srw_forward(ctypes.byref(d), ctypes.byref(t), ctypes.byref(o), None, 0, None)
    assert st == C.SRW_EINVAL
    assert C.load_library().srw_forward(ctypes.byref(d), None, None, None, 0, None) == C.SRW_EINVAL


def test_workspace_sizes(C):
    # generic kernels: no workspace for the v4.1 gate
    assert C.workspace_size(_desc(C, flags=C.SRW_FLAG_NO_FAST)) == 0
    # matrix-core path (T=16, D=64, dr=32, N=100): packed W^T of ceil(N/32)
    # tiles, per-N-split moments, per-token tau, and partial out / per-token
    # partials for S = 3 splits (one 128-token tile, a split per 32-unit tile,
    # 3 whole tiles)
    al = lambda b: (b + 255) // 256 * 256  # noqa: E731
    S, T, D = 3, 16, 64
    want = (al(4 * 32 * D * 2) + al(S * T * 2 * 4) + al(T * 4) + al(S * T * D * 4)
            + al(S * T * 4 * 4))
    assert C.workspace_size(_desc(C)) == want
    # d_route == d_model: also the bf16 scores the main kernel streams (8 KB
    # per 128-token tile and 32-unit tile)
    assert C.workspace_size(_desc(C, d_route=64)) == want + al(1 * 4 * 8192)
    # the v4.0.1 gate on the matrix cores: also forward-normalised R and W
    # copies (bf16) and the rows' s_std
    d = _desc(C, gate=C.SRW_GATE_GELU_V401)
    assert C.workspace_size(d) == want + 2 * al(100 * 64 * 2) + al(T * 4)
    # ... in fp32 on the fp32 matrix cores: the v4.1 layout plus forward-
    # normalised R and W (fp32) and the rows' s_std
    f32 = C.workspace_size(_desc(C, dtype=C.SRW_F32))
    d = _desc(C, gate=C.SRW_GATE_GELU_V401, dtype=C.SRW_F32)
    assert C.workspace_size(d) == f32 + 2 * al(100 * 64 * 4) + al(T * 4)
    # ... on the generic kernels (f32): the two row copies only
    d = _desc(C, gate=C.SRW_GATE_GELU_V401, dtype=C.SRW_F32, flags=C.SRW_FLAG_NO_FAST)
    assert C.workspace_size(d) == 2 * 100 * 64 * 4


def test_gate_out_sizes_the_tiled_families(C):
    """SRW_FLAG_GATE_OUT: the dense gate comes from the tiled gate epilogue
    (bf16 widths multiples of 64, fp32 of 32), else the generic kernels."""
    bf_tiled = C.workspace_size(_desc(C, d_route=64, flags=C.SRW_FLAG_TILED))
    assert bf_tiled > 0
    assert C.workspace_size(_desc(C, d_route=64, flags=C.SRW_FLAG_GATE_OUT)) == bf_tiled
    # d_route = 32 has no bf16 tiled kernel: the generic kernels, no workspace
    assert C.workspace_size(_desc(C, flags=C.SRW_FLAG_GATE_OUT)) == 0
    f32 = C.workspace_size(_desc(C, dtype=C.SRW_F32))
    assert f32 > 0 and C.workspace_size(_desc(C, dtype=C.SRW_F32, flags=C.SRW_FLAG_GATE_OUT)) == f32


@pytest.mark.parametrize("shape", [(384, 384, 1, 0), (384, 128, 2, 0), (1024, 1024, 1, 0),
                                   (384, 384, 1, 0x20), (128, 64, 1, 0)])
def test_no_tokens_need_no_workspace(C, shape):
    """T = 0 sizes to zero bytes on every family, forward and backward (the
    sizing divides nothing by T)."""
    D, dr, R, flags = shape
    d = _desc(C, T=0, d_model=D, d_route=dr, n_routes=R, n_units=300, flags=flags)
    assert C.workspace_size(d) == 0
    assert C.backward_workspace_size(d) == 0
    d.T = 1
    assert C.workspace_size(d) > 0 and C.backward_workspace_size(d) > 0


def test_batch_workspace_is_the_aligned_sum(C):
    """srw_workspace_size_batch: call i's workspace slice follows the 256-byte
    aligned slices of calls 0 .. i-1 (srw_forward_batch)."""
    al = lambda b: (b + 255) // 256 * 256  # noqa: E731
    descs = (C.SrwDesc * 3)(_desc(C), _desc(C, d_route=64), _desc(C, T=100, n_units=777))
    want = sum(al(C.workspace_size(d)) for d in descs)
    assert C.workspace_size_batch(descs) == want
    assert C.workspace_size_batch((C.SrwDesc * 1)(descs[1])) == al(C.workspace_size(descs[1]))


def test_batch_arguments_checked_before_any_launch(C):
    lib = C.load_library()
    n = ctypes.c_size_t(0)
    five = (C.SrwDesc * 5)(*[_desc(C)] * 5)
    assert lib.srw_workspace_size_batch(0, five, ctypes.byref(n)) == C.SRW_EINVAL
    assert lib.srw_workspace_size_batch(5, five, ctypes.byref(n)) == C.SRW_EINVAL
    bad = (C.SrwDesc * 2)(_desc(C), _desc(C, d_model=0))
    assert lib.srw_workspace_size_batch(2, bad, ctypes.byref(n)) == C.SRW_EINVAL
    t, o = (C.SrwTensors * 2)(), (C.SrwOutputs * 2)()
    good = (C.SrwDesc * 2)(_desc(C), _desc(C))
    # null tensors, then too small a workspace: refused on the host
    assert lib.srw_forward_batch(2, good, t, o, None, 0, None) in (C.SRW_EINVAL, C.SRW_EWORKSPACE)
    assert lib.srw_forward_batch(2, good, None, o, None, 0, None) == C.SRW_EINVAL


def test_noalloc_refusals_before_any_launch(C):
    """srw_forward_noalloc checks its descriptor, the pool-cached flag and the
    scratch size on the host: nothing reaches a GPU."""
    lib = C.load_library()
    t, o = C.SrwTensors(), C.SrwOutputs()
    d = _desc(C, d_model=0)
    assert lib.srw_forward_noalloc(ctypes.byref(d), ctypes.byref(t), ctypes.byref(o), None) == C.SRW_EINVAL
    d = _desc(C, flags=C.SRW_FLAG_POOL_CACHED)
    assert lib.srw_forward_noalloc(ctypes.byref(d), ctypes.byref(t), ctypes.byref(o), None) == C.SRW_EINVAL
    # configs[0] at T = 4096: ~264 MiB of workspace, beyond the 64 MiB scratch
    d = _desc(C, T=4096, d_model=384, d_route=384, n_units=25200, chunk_size=12600)
    assert C.workspace_size(d) > C.NOALLOC_SCRATCH_BYTES
    assert lib.srw_forward_noalloc(ctypes.byref(d), ctypes.byref(t), ctypes.byref(o), None) == C.SRW_ESCRATCH
    # a decode-sized Know call (64 rows, d_route 128) fits
    d = _desc(C, T=64, d_model=384, d_route=128, n_units=25200, chunk_size=12600)
    assert 0 < C.workspace_size(d) <= C.NOALLOC_SCRATCH_BYTES
    # no tokens: nothing to compute, no scratch looked up
    d = _desc(C, T=0)
    assert lib.srw_forward_noalloc(ctypes.byref(d), ctypes.byref(t), ctypes.byref(o), None) == C.SRW_OK


def test_status_strings(C):
    lib = C.load_library()
    for s in range(6):
        assert lib.srw_status_string(s).decode().startswith("SRW_")
    with pytest.raises(C.SrwError):
        C.check(C.SRW_EINVAL)


def test_wrapper_refuses_cpu_tensors(pkg):
    import torch
    x = torch.zeros(4, 8)
    with pytest.raises(ValueError):
        pkg.srw_forward(x, x, torch.zeros(3, 8), torch.zeros(4, 1), torch.zeros(3, 8), torch.zeros(3, 8))


def test_mesh_larger_than_one_device_refused(pkg):
    class Mesh:
        shape = {"data": 1, "model": 2}
    with pytest.raises(NotImplementedError):
        pkg.make_sharded_srw(Mesh())
    pkg.make_sharded_srw(None)


def test_v401_backward_workspace_holds_the_normalised_rows(C):
    """srw_backward_workspace_size with the v4.0.1 gate: the v4.1 layout plus
    the forward-normalised read and write rows (bf16, N x D each) and the
    per-row sums of dm z ([N64 / 64][T] fp32)."""
    al = lambda b: (b + 255) // 256 * 256  # noqa: E731
    T, D, dr, N = 16, 64, 64, 100
    base = C.backward_workspace_size(_desc(C, T=T, d_model=D, d_route=dr, n_units=N))
    gl = C.backward_workspace_size(_desc(C, T=T, d_model=D, d_route=dr, n_units=N, gate=C.SRW_GATE_GELU_V401))
    N64 = (N + 63) // 64 * 64
    assert gl == base + 2 * al(N * D * 2) + al(N64 // 64 * T * 4)
    # the v4.0.1 function has no dead penalty: a cotangent for it is refused
    # before any launch (no tensors are touched)
    d = _desc(C, T=T, d_model=D, d_route=dr, n_units=N, gate=C.SRW_GATE_GELU_V401)
    cot = C.SrwCotangents(256, 256, 0.0, 0.5, None, None)
    t = C.SrwTensors(256, 256, 256, 256, 256, 256)
    g = C.SrwGrads(256, 256, 256, 256, 256, 256, None)
    st = C.load_library().srw_backward(ctypes.byref(d), ctypes.byref(t), ctypes.byref(cot), ctypes.byref(g),
                                       None, 0, None)
    assert st == C.SRW_EINVAL
