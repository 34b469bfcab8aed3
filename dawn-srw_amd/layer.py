"""Host wrapper of ``srw_forward``: torch tensors in, torch tensors out.

This is the single place where tensors cross into libsrw_amd.so
(``SrwPlan``; ``srw_forward`` is a one-shot plan).  It checks
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


class SrwPlan:
    """One bound ``srw_forward`` call: inputs checked, outputs and workspace
    allocated, and the C descriptor structs built once, so that ``launch()``
    is a single C call (benchmarks, loops over the same buffers).

    The arguments are those of :func:`srw_forward`.  The input tensors are
    held by reference; overwrite them in place to feed new data.
    """

    def __init__(self, x, h, emb, tau_offset, read, write, *, gate: str = "v41",
                 stats: str = "onepass", consts: GateConfig = GateConfig(),
                 scale: float = 1.0, chunk_size: int = 0, diag: bool = False,
                 want_mask: bool = True, emulate: bool = False,
                 sparse_skip: bool = False, force_generic: bool = False,
                 want_gate: bool = False, tiled: bool = False):
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
        if gate not in _GATES:
            raise ValueError(f"gate must be one of {sorted(_GATES)}")
        if stats not in _STATS:
            raise ValueError(f"stats must be one of {sorted(_STATS)}")

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
                      | (C.SRW_FLAG_NO_FAST if force_generic else 0)
                      | (C.SRW_FLAG_TILED if tiled else 0)
                      | (C.SRW_FLAG_GATE_OUT if want_gate else 0))

        words = (N + 63) // 64
        self.out = torch.empty((T, R, D), dtype=dt, device=dev)
        self.gate_sum = torch.empty((T, R), dtype=torch.float32, device=dev)
        self.den = torch.empty((T, R), dtype=torch.float32, device=dev)
        self.n_active = torch.empty((T, R), dtype=torch.int32, device=dev)
        self.pass_mask = (torch.empty((T, R, words), dtype=torch.int64, device=dev)
                          if want_mask else None)
        self.token_diag = (torch.empty((T, R, len(C.TDIAG)), dtype=torch.float32, device=dev)
                           if diag else None)
        self.unit_diag = (torch.empty((N, len(C.UDIAG)), dtype=torch.float32, device=dev)
                          if diag else None)
        self.gate = (torch.empty((T, R, N), dtype=torch.float32, device=dev)
                     if want_gate else None)
        self.ws_bytes = C.workspace_size(desc)
        self.workspace = torch.empty(max(self.ws_bytes, 1), dtype=torch.uint8, device=dev)

        self.inputs = (x, h, emb, tau_offset, read, write)
        self.device = dev
        self.shape = dict(T=T, D=D, dr=dr, N=N, R=R)
        self._desc = desc
        self._tens = C.SrwTensors(_ptr(x), _ptr(x if h_is_x else h), _ptr(emb),
                                  _ptr(tau_offset), _ptr(read), _ptr(write))
        self._outs = C.SrwOutputs(_ptr(self.out), _ptr(self.gate_sum), _ptr(self.den),
                                  _ptr(self.n_active), _ptr(self.pass_mask),
                                  _ptr(self.token_diag), _ptr(self.unit_diag), _ptr(self.gate))
        self._lib = C.load_library()
        self.path = None

    def launch(self, stream=None, pool_cached: bool = False) -> None:
        """Enqueue the call on ``stream`` (default: torch's current stream).

        ``pool_cached=True`` declares that ``emb``, ``read`` and ``write`` are
        unchanged since this plan's previous launch (decode steps over one
        pool): the pool-derived data kept in the workspace (packed W^T, Gram
        statistics) is reused instead of rebuilt.
        """
        if stream is None:
            with torch.cuda.device(self.device):
                stream = torch.cuda.current_stream(self.device)
        if pool_cached and self.path is None:
            raise ValueError("pool_cached needs an earlier launch of this plan")
        base = self._desc.flags
        if pool_cached:
            self._desc.flags = base | C.SRW_FLAG_POOL_CACHED
        try:
            C.check(self._lib.srw_forward(
                ctypes.byref(self._desc), ctypes.byref(self._tens), ctypes.byref(self._outs),
                _ptr(self.workspace), ctypes.c_size_t(self.ws_bytes),
                ctypes.c_void_p(stream.cuda_stream)))
        finally:
            self._desc.flags = base
        self.path = C.last_path()

    def results(self) -> dict:
        return dict(out=self.out, gate_sum=self.gate_sum, den=self.den,
                    n_active=self.n_active, pass_mask=self.pass_mask,
                    token_diag=self.token_diag, unit_diag=self.unit_diag, gate=self.gate,
                    path=self.path, workspace=self.workspace)


class SrwBatchPlan:
    """Several bound calls enqueued together through ``srw_forward_batch``.

    The plans' descriptors, tensors and outputs are taken over (each plan's
    results land in its own output tensors, as after its own launch); the
    workspace is one batch workspace, sliced in plan order, so the plans' own
    workspaces are not used.  Calls that all take the same kernel
    instantiations (the QK and V calls of a layer, at decode or prefill
    sizes) run as one launch per stage; others run one after the other --
    the results equal separate launches bit for bit either way.
    """

    def __init__(self, plans):
        plans = list(plans)
        if not 1 <= len(plans) <= C.MAX_BATCH:
            raise ValueError(f"a batch holds 1 to {C.MAX_BATCH} plans, got {len(plans)}")
        dev = plans[0].device
        if any(p.device != dev for p in plans):
            raise ValueError("the plans of a batch share one device")
        n = len(plans)
        self.plans = plans
        self.device = dev
        self._descs = (C.SrwDesc * n)(*[p._desc for p in plans])
        self._tens = (C.SrwTensors * n)(*[p._tens for p in plans])
        self._outs = (C.SrwOutputs * n)(*[p._outs for p in plans])
        self.ws_bytes = C.workspace_size_batch(self._descs)
        self.workspace = torch.empty(max(self.ws_bytes, 1), dtype=torch.uint8, device=dev)
        self._lib = C.load_library()
        self.path = None

    def launch(self, stream=None, pool_cached: bool = False) -> None:
        """Enqueue the calls on ``stream`` (default: torch's current stream);
        ``pool_cached`` as in :meth:`SrwPlan.launch`, relative to this batch's
        previous launch."""
        if stream is None:
            with torch.cuda.device(self.device):
                stream = torch.cuda.current_stream(self.device)
        if pool_cached and self.path is None:
            raise ValueError("pool_cached needs an earlier launch of this batch")
        base = [d.flags for d in self._descs]
        if pool_cached:
            for d in self._descs:
                d.flags = d.flags | C.SRW_FLAG_POOL_CACHED
        try:
            C.check(self._lib.srw_forward_batch(
                len(self.plans), self._descs, self._tens, self._outs,
                _ptr(self.workspace), ctypes.c_size_t(self.ws_bytes),
                ctypes.c_void_p(stream.cuda_stream)))
        finally:
            for d, f in zip(self._descs, base):
                d.flags = f
        self.path = C.last_path()
        for p in self.plans:
            p.path = self.path


def srw_forward(x, h, emb, tau_offset, read, write, *, gate: str = "v41",
                stats: str = "onepass", consts: GateConfig = GateConfig(),
                scale: float = 1.0, chunk_size: int = 0, diag: bool = False,
                want_mask: bool = True, emulate: bool = False,
                sparse_skip: bool = False, force_generic: bool = False,
                want_gate: bool = False, tiled: bool = False) -> dict:
    """One SRW layer forward on the GPU.

    x [T, D]; h [T, R, dr] (R = 1 or 2) or the tensor ``x`` itself (R = 1,
    dr = D); emb [N, dr]; tau_offset [T, R] float32; read, write [N, D].
    x, h, emb, read and write share one dtype (float32 or bfloat16), all on
    one CUDA (HIP) device, contiguous.

    Options: ``gate`` "v41" | "gelu_v401"; ``stats`` "onepass" (moments of
    the rounded scores, fused_gate_srw) | "centered" (two-pass,
    _srw_inference) | "gram" (closed form from E^T E); ``chunk_size`` the
    reference's N-chunk (its partial write GEMMs are rounded to bf16 per
    chunk); ``scale`` multiplies out after the den division; ``tiled`` runs
    the tiled-GEMM kernels (the gated product materialised in the workspace)
    even where a fused kernel exists -- they serve d_model > 384 anyway.

    Returns a dict: out [T, R, D] (input dtype), gate_sum / den [T, R] f32,
    n_active [T, R] int32, pass_mask [T, R, ceil(N/64)] int64 (bit n % 64 of
    word n // 64) or None, token_diag [T, R, 14] / unit_diag [N, 2] f32 when
    ``diag``, gate [T, R, N] f32 when ``want_gate`` (every unit's gate; such a
    call runs the generic kernels), and ``path`` (the kernel family used).
    """
    plan = SrwPlan(x, h, emb, tau_offset, read, write, gate=gate, stats=stats,
                   consts=consts, scale=scale, chunk_size=chunk_size, diag=diag,
                   want_mask=want_mask, emulate=emulate, sparse_skip=sparse_skip,
                   force_generic=force_generic, want_gate=want_gate, tiled=tiled)
    plan.launch()
    return plan.results()


class SrwBackwardPlan:
    """One bound ``srw_backward`` call: inputs checked, gradients and the
    workspace allocated and the C structs built once, so that ``launch()``
    is a single C call.  Arguments as :func:`srw_backward`; the tensors are
    held by reference (overwrite them in place to feed new data)."""

    def __init__(self, x, h, emb, tau_offset, read, write, out, d_out, d_score_lb: float = 0.0,
                 d_dead_penalty: float = 0.0, *, consts: GateConfig = GateConfig(),
                 scale: float = 1.0, den=None, unit_diag=None, gate: str = "v41"):
        if gate not in _GATES:
            raise ValueError(f"gate must be one of {sorted(_GATES)}")
        if x.dim() != 2:
            raise ValueError("x must be [T, D]")
        T, D = x.shape
        dev = x.device
        if dev.type != "cuda":
            raise ValueError("srw_backward runs on a HIP device; got " + str(dev))
        if x.dtype != torch.bfloat16:
            raise TypeError("srw_backward takes bfloat16 inputs")
        h_is_x = h is x
        if h_is_x:
            R, dr = 1, D
        else:
            if h.dim() != 3 or h.shape[1] not in (1, 2):
                raise ValueError("h must be [T, R, d_route] with R = 1 or 2")
            R, dr = h.shape[1], h.shape[2]
            _check_dev("h", h, dev, x.dtype, (T, R, dr))
        N = emb.shape[0]
        _check_dev("x", x, dev, x.dtype)
        _check_dev("emb", emb, dev, x.dtype, (N, dr))
        _check_dev("tau_offset", tau_offset, dev, torch.float32, (T, R))
        _check_dev("read", read, dev, x.dtype, (N, D))
        _check_dev("write", write, dev, x.dtype, (N, D))
        _check_dev("out", out, dev, x.dtype, (T, R, D))
        _check_dev("d_out", d_out, dev, torch.float32, (T, R, D))
        if (den is None) != (unit_diag is None):
            raise ValueError("den and unit_diag (the forward's residuals) go together")
        if den is not None:
            _check_dev("den", den, dev, torch.float32, (T, R))
            _check_dev("unit_diag", unit_diag, dev, torch.float32, (N, len(C.UDIAG)))
        desc = C.desc_init()
        desc.T, desc.d_model, desc.d_route, desc.n_units = T, D, dr, N
        desc.n_routes = R
        desc.dtype = C.SRW_BF16
        desc.gate = _GATES[gate]
        desc.sharpness = consts.sharpness
        desc.act_threshold = consts.activation_threshold
        desc.act_cutoff = consts.activation_cutoff
        desc.epsilon = consts.epsilon
        desc.max_intensity = consts.max_intensity
        desc.dead_threshold = consts.dead_threshold
        desc.scale = scale
        f32 = dict(dtype=torch.float32, device=dev)
        self.grads = dict(dx=torch.empty(T, D, **f32), dh=torch.empty(T, R, dr, **f32),
                          demb=torch.empty(N, dr, **f32), dtau_offset=torch.empty(T, R, **f32),
                          dread=torch.empty(N, D, **f32), dwrite=torch.empty(N, D, **f32),
                          dscale=torch.empty((), **f32))
        self.ws_bytes = C.backward_workspace_size(desc)
        self.workspace = torch.empty(max(self.ws_bytes, 1), dtype=torch.uint8, device=dev)
        self.inputs = (x, h, emb, tau_offset, read, write, out, d_out, den, unit_diag)
        self.device = dev
        self._desc = desc
        self._tens = C.SrwTensors(_ptr(x), _ptr(x if h_is_x else h), _ptr(emb), _ptr(tau_offset),
                                  _ptr(read), _ptr(write))
        self._cot = C.SrwCotangents(_ptr(d_out), _ptr(out), float(d_score_lb), float(d_dead_penalty),
                                    _ptr(den), _ptr(unit_diag))
        self._g = C.SrwGrads(*(_ptr(self.grads[k]) for k in
                               ("dx", "dh", "demb", "dtau_offset", "dread", "dwrite", "dscale")))
        self._lib = C.load_library()
        self.path = None

    def launch(self, stream=None) -> None:
        if stream is None:
            with torch.cuda.device(self.device):
                stream = torch.cuda.current_stream(self.device)
        C.check(self._lib.srw_backward(
            ctypes.byref(self._desc), ctypes.byref(self._tens), ctypes.byref(self._cot),
            ctypes.byref(self._g), _ptr(self.workspace), ctypes.c_size_t(self.ws_bytes),
            ctypes.c_void_p(stream.cuda_stream)))
        self.path = C.last_path()

    def results(self) -> dict:
        return dict(self.grads, path=self.path, workspace_bytes=self.ws_bytes)


def srw_backward(x, h, emb, tau_offset, read, write, out, d_out, d_score_lb: float = 0.0,
                 d_dead_penalty: float = 0.0, *, consts: GateConfig = GateConfig(),
                 scale: float = 1.0, stream=None, den=None, unit_diag=None, gate: str = "v41") -> dict:
    """Reverse-mode derivative of one srw_forward call (the VJP of
    fused_gate_srw that the reference's train_step takes with
    jax.value_and_grad, scripts/train_jax.py:548-726).

    Inputs as :func:`srw_forward` (bf16; h [T, R, dr] with R = 1, or 2 for
    the paired QK routes of fused_gate_srw_paired, v41:640-909, or x itself),
    ``out`` [T, R, D] the forward's output on them, ``d_out`` the cotangent
    of ``out`` (float32, same shape), ``d_score_lb`` / ``d_dead_penalty`` the
    cotangents of the score_lb and dead_penalty outputs (v41:477-483,
    543-552).  Returns float32 gradients dx [T, D], dh [T, R, dr], demb
    [N, dr], dtau_offset [T, R], dread / dwrite [N, D] and dscale [] (of
    ``scale``, which multiplies out: the caller's *_scale, v41:1044-1053,
    1175); when ``h is x`` the total gradient of x is dx + dh[:, 0].
    ``den`` [T, R] and ``unit_diag`` [N, 2] (both or neither): the same
    forward call's den and unit diagnostics (a ``diag=True`` call, as the
    drop-in's forward makes), which spare the backward its own pass over the
    scores for them.  ``gate`` "gelu_v401": the VJP of the v4.0.1 fused
    function (models/legacy/dawn_spatial_v401_exp.py:229-554), which has no
    dead_penalty (``d_dead_penalty`` must be 0).
    """
    plan = SrwBackwardPlan(x, h, emb, tau_offset, read, write, out, d_out, d_score_lb,
                           d_dead_penalty, consts=consts, scale=scale, den=den, unit_diag=unit_diag,
                           gate=gate)
    plan.launch(stream)
    return plan.results()
