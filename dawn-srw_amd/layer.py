"""Host wrapper of ``srw_forward``: torch tensors in, torch tensors out.

This is the single place where tensors cross into libsrw_amd.so.  It checks
shapes, dtypes and devices, allocates the outputs and the workspace with
torch's caching allocator, and enqueues the call on torch's current stream.
Every computation runs in the library's HIP kernels; there is no CPU or
PyTorch fallback.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _capi as C

_DTYPES = {torch.float32: C.SRW_F32, torch.bfloat16: C.SRW_BF16}
_GATES = {"v41": C.SRW_GATE_V41, "gelu_v401": C.SRW_GATE_GELU_V401}
_STATS = {"onepass": C.SRW_STATS_ONEPASS, "centered": C.SRW_STATS_CENTERED,
          "gram": C.SRW_STATS_GRAM}


@dataclass(frozen=True)
class GateConfig:
    """Gate constants of make_sharded_srw (models/dawn_spatial_v41_exp.py:297-301, 352-357)."""
    sharpness: float = 500.0
    activation_threshold: float = 0.5
    activation_cutoff: float = 0.01
    epsilon: float = 1e-4
    max_intensity: float = 10.0
    dead_threshold: float = 0.01


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def _check_dev(name, t, dev, dtype=None, shape=None):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.device != dev:
        raise ValueError(f"{name} is on {t.device}, expected {dev}")
    if dtype is not None and t.dtype != dtype:
        raise TypeError(f"{name} has dtype {t.dtype}, expected {dtype}")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def srw_forward(x, h, emb, tau_offset, read, write, *, gate: str = "v41",
                stats: str = "onepass", consts: GateConfig = GateConfig(),
                scale: float = 1.0, chunk_size: int = 0, diag: bool = False,
                want_mask: bool = True, emulate: bool = False,
                sparse_skip: bool = False, force_generic: bool = False) -> dict:
    """One SRW layer forward on the GPU.

    x [T, D]; h [T, R, dr] (R = 1 or 2) or the tensor ``x`` itself (R = 1,
    dr = D); emb [N, dr]; tau_offset [T, R] float32; read, write [N, D].
    x, h, emb, read and write share one dtype (float32 or bfloat16), all on
    one CUDA (HIP) device, contiguous.

    Returns a dict: out [T, R, D] (input dtype), gate_sum / den [T, R] f32,
    n_active [T, R] int32, pass_mask [T, R, ceil(N/64)] int64 (bit n % 64 of
    word n // 64) or None, token_diag [T, R, 14] / unit_diag [N, 2] f32 when
    ``diag``, and ``path`` (the kernel family used).
    """
    if x.dim() != 2:
        raise ValueError("x must be [T, D]")
    T, D = x.shape
    dev = x.device
    if dev.type != "cuda":
        raise ValueError("srw_forward runs on a HIP device; got " + str(dev))
    dt = x.dtype
    if dt not in _DTYPES:
        raise TypeError(f"unsupported dtype {dt}")
    h_is_x = h is x
    if h_is_x:
        R, dr = 1, D
    else:
        if h.dim() != 3:
            raise ValueError("h must be [T, R, d_route]")
        R, dr = h.shape[1], h.shape[2]
        _check_dev("h", h, dev, dt, (T, R, dr))
    N = emb.shape[0]
    _check_dev("x", x, dev, dt)
    _check_dev("emb", emb, dev, dt, (N, dr))
    _check_dev("tau_offset", tau_offset, dev, torch.float32, (T, R))
    _check_dev("read", read, dev, dt, (N, D))
    _check_dev("write", write, dev, dt, (N, D))

    desc = C.desc_init()
    desc.T, desc.d_model, desc.d_route, desc.n_units = T, D, dr, N
    desc.n_routes = R
    desc.dtype = _DTYPES[dt]
    desc.gate = _GATES[gate]
    desc.stats_mode = _STATS[stats]
    desc.sharpness = consts.sharpness
    desc.act_threshold = consts.activation_threshold
    desc.act_cutoff = consts.activation_cutoff
    desc.epsilon = consts.epsilon
    desc.max_intensity = consts.max_intensity
    desc.dead_threshold = consts.dead_threshold
    desc.scale = scale
    desc.chunk_size = int(chunk_size)
    desc.flags = ((C.SRW_FLAG_DIAG if diag else 0) | (C.SRW_FLAG_EMULATE if emulate else 0)
                  | (C.SRW_FLAG_SPARSE_SKIP if sparse_skip else 0)
                  | (C.SRW_FLAG_NO_FAST if force_generic else 0))

    words = (N + 63) // 64
    out = torch.empty((T, R, D), dtype=dt, device=dev)
    gate_sum = torch.empty((T, R), dtype=torch.float32, device=dev)
    den = torch.empty((T, R), dtype=torch.float32, device=dev)
    n_active = torch.empty((T, R), dtype=torch.int32, device=dev)
    mask = torch.empty((T, R, words), dtype=torch.int64, device=dev) if want_mask else None
    tdiag = torch.empty((T, R, len(C.TDIAG)), dtype=torch.float32, device=dev) if diag else None
    udiag = torch.empty((N, len(C.UDIAG)), dtype=torch.float32, device=dev) if diag else None

    ws_bytes = C.workspace_size(desc)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)

    tens = C.SrwTensors(_ptr(x), _ptr(x if h_is_x else h), _ptr(emb), _ptr(tau_offset),
                        _ptr(read), _ptr(write))
    outs = C.SrwOutputs(_ptr(out), _ptr(gate_sum), _ptr(den), _ptr(n_active), _ptr(mask),
                        _ptr(tdiag), _ptr(udiag))
    with torch.cuda.device(dev):
        stream = torch.cuda.current_stream(dev).cuda_stream
        C.check(C.load_library().srw_forward(
            ctypes.byref(desc), ctypes.byref(tens), ctypes.byref(outs),
            _ptr(ws), ctypes.c_size_t(ws_bytes), ctypes.c_void_p(stream)))
    return dict(out=out, gate_sum=gate_sum, den=den, n_active=n_active,
                pass_mask=mask, token_diag=tdiag, unit_diag=udiag,
                path=C.last_path(), workspace=ws)
