"""GPU: srw_forward_noalloc (the entry point without a workspace argument,
whose workspace is the library's per-GPU static scratch) against srw_forward
with a caller workspace, through the C ABI.

Both run the same kernels on the same inputs, so the outputs must be equal
bit for bit.  Each case makes two no-allocation calls in a row on one GPU,
the second with fewer tokens, so that the scratch holds the first call's
data when the second starts.  A call that needs more than the scratch
returns SRW_ESCRATCH and writes nothing.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

BF = torch.bfloat16
KEYS = ("out", "gate_sum", "den", "n_active", "pass_mask")


def _plan(pkg, shape, T, seed):
    inp = pkg.inputs.make_pool_inputs(shape, seed=seed, T=T)
    if shape.pass_target is not None:
        inp["tau_offset"].fill_(pkg.inputs.calibrate_tau_offset(inp, shape.pass_target))
    dev = torch.device("cuda:0")
    x = inp["x"].to(BF).to(dev)
    h = x if shape.h_is_x else inp["h"].to(BF).to(dev)
    _, cs = pkg.chunk_plan(shape.N, 12500)
    return pkg.SrwPlan(x, h, inp["emb"].to(BF).to(dev), inp["tau_offset"].to(dev), inp["read"].to(BF).to(dev),
                       inp["write"].to(BF).to(dev), chunk_size=cs, want_mask=True)


def _noalloc(pkg, plan, stream):
    """The plan's call through srw_forward_noalloc into fresh outputs
    (pre-filled with a sentinel)."""
    C = pkg._capi
    outs = {k: torch.full_like(getattr(plan, k), -7) for k in KEYS}
    o = C.SrwOutputs(*(ctypes.c_void_p(outs[k].data_ptr()) for k in KEYS), None, None, None)
    st = C.load_library().srw_forward_noalloc(ctypes.byref(plan._desc), ctypes.byref(plan._tens),
                                             ctypes.byref(o), ctypes.c_void_p(stream.cuda_stream))
    return st, outs


def test_noalloc_first_call_under_graph_capture(pkg, dev):
    """The first srw_forward_noalloc call of the process on this GPU -- the
    one that looks up the scratch's device address -- made while the stream
    is being captured into a graph (torch.cuda.graph, global capture mode).
    The graph is replayed three times, with eager work and a synchronisation
    between the replays and the outputs refilled with a sentinel before
    each; every replay equals srw_forward with a caller workspace bit for
    bit.  (This test comes first in the file so that no other no-allocation
    call precedes it.)"""
    shape = pkg.inputs.CONFIGS["decode_qk"]
    print(f"[gpu] noalloc first call under capture: decode_qk T64 N{shape.N} R{shape.routes}", flush=True)
    plan = _plan(pkg, shape, 64, seed=9)
    C = pkg._capi
    eager = torch.cuda.current_stream(dev)
    plan.launch(eager)                     # the reference result; also loads the kernels
    torch.cuda.synchronize()
    want = {k: getattr(plan, k).clone() for k in KEYS}
    outs = {k: torch.full_like(want[k], -7) for k in KEYS}
    o = C.SrwOutputs(*(ctypes.c_void_p(outs[k].data_ptr()) for k in KEYS), None, None, None)
    lib = C.load_library()
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream(dev)
    cap.wait_stream(eager)
    with torch.cuda.graph(graph, stream=cap):
        st = lib.srw_forward_noalloc(ctypes.byref(plan._desc), ctypes.byref(plan._tens), ctypes.byref(o),
                                     ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream))
    torch.cuda.synchronize()
    assert st == C.SRW_OK, lib.srw_status_string(st)
    for rep in range(3):
        for k in KEYS:
            outs[k].fill_(-7)
        plan.launch(eager)                 # eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for k in KEYS:
            assert torch.equal(outs[k], want[k]), (rep, k)
        print(f"  replay {rep + 1}: equal bit for bit", flush=True)


@pytest.mark.parametrize("key,sizes", [("decode_know", (64, 16)), ("v", (256, 100)), ("decode_qk", (64, 7))])
def test_noalloc_equals_srw_forward(pkg, dev, key, sizes):
    shape = pkg.inputs.CONFIGS[key]
    stream = torch.cuda.current_stream(dev)
    for i, T in enumerate(sizes):
        print(f"[gpu] noalloc {key} call {i + 1}: T{T} D{shape.D} dr{shape.dr} N{shape.N} R{shape.routes}",
              flush=True)
        plan = _plan(pkg, shape, T, seed=3 + i)
        assert plan.ws_bytes <= pkg._capi.NOALLOC_SCRATCH_BYTES
        plan.launch(stream)
        torch.cuda.synchronize()
        st, outs = _noalloc(pkg, plan, stream)
        torch.cuda.synchronize()
        assert st == pkg._capi.SRW_OK, pkg._capi.load_library().srw_status_string(st)
        for k in KEYS:
            assert torch.equal(outs[k], getattr(plan, k)), (key, T, k)
        print(f"  path {pkg._capi.last_path()}: equal bit for bit", flush=True)


def test_noalloc_refuses_calls_beyond_the_scratch(pkg, dev):
    """configs[0] at T = 4096 needs ~264 MiB of workspace: SRW_ESCRATCH,
    nothing launched, outputs untouched."""
    shape = pkg.inputs.CONFIGS["know"]
    print(f"[gpu] noalloc refusal T{shape.T} N{shape.N}", flush=True)
    plan = _plan(pkg, shape, shape.T, seed=0)
    assert plan.ws_bytes > pkg._capi.NOALLOC_SCRATCH_BYTES
    stream = torch.cuda.current_stream(dev)
    st, outs = _noalloc(pkg, plan, stream)
    torch.cuda.synchronize()
    assert st == pkg._capi.SRW_ESCRATCH
    assert "SRW_ESCRATCH" in pkg._capi.load_library().srw_status_string(st).decode()
    for k in KEYS:
        assert bool((outs[k] == -7).all()), k
