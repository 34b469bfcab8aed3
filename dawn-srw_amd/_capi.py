"""ctypes binding of libsrw_amd.so (the C ABI declared in include/srw_amd.h).

The library is loaded from ``<package>/lib/libsrw_amd.so``, built in-tree by
``__graft_entry__.build()`` (``make -C dawn-srw_amd/csrc``).  There is no
fallback: if the library is missing every entry point raises
``SrwLibraryError``.

torch is imported before the library is loaded so that the library binds to
the HIP runtime PyTorch-ROCm already mapped (one runtime per process; the
stream handles torch hands out are only valid there).
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must precede loading the HIP library)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "libsrw_amd.so")
ABI_VERSION = 7
MAX_BATCH = 4          # SRW_MAX_BATCH

# srw_status_t
SRW_OK, SRW_EINVAL, SRW_EUNSUPPORTED, SRW_EHIP, SRW_EWORKSPACE, SRW_ESCRATCH = range(6)
# bytes of srw_forward_noalloc's per-GPU scratch (SRW_NOALLOC_SCRATCH_BYTES)
NOALLOC_SCRATCH_BYTES = 64 << 20
# srw_dtype_t
SRW_F32, SRW_BF16 = 0, 1
# srw_gate_t
SRW_GATE_V41, SRW_GATE_GELU_V401 = 0, 1
# srw_stats_mode_t
SRW_STATS_ONEPASS, SRW_STATS_CENTERED, SRW_STATS_GRAM = 0, 1, 2
# flags
SRW_FLAG_DIAG = 0x1
SRW_FLAG_EMULATE = 0x2
SRW_FLAG_SPARSE_SKIP = 0x4
SRW_FLAG_NO_FAST = 0x8
SRW_FLAG_POOL_CACHED = 0x10
SRW_FLAG_TILED = 0x20
SRW_FLAG_GATE_OUT = 0x40

# token_diag columns (SRW_TDIAG_*) and unit_diag columns (SRW_UDIAG_*)
TDIAG = (
    "s_mean", "s_std", "tau", "sum_s3", "sum_s4", "gate_max", "int_sum",
    "n_strong", "n_boundary", "n_band075", "n_band030", "g_log_g", "int_max",
    "n_int_cap",
)
TDIAG_INDEX = {k: i for i, k in enumerate(TDIAG)}
UDIAG = ("score_sum", "gate_max")

# Every symbol include/srw_amd.h declares.
EXPORTED_SYMBOLS = (
    "srw_abi_version", "srw_status_string", "srw_desc_init",
    "srw_workspace_size", "srw_forward", "srw_last_path",
    "srw_set_kernel_events", "srw_backward_workspace_size", "srw_backward",
    "srw_workspace_size_batch", "srw_forward_batch", "srw_forward_noalloc",
)


class SrwDesc(ctypes.Structure):
    _fields_ = [
        ("T", ctypes.c_int64), ("d_model", ctypes.c_int64),
        ("d_route", ctypes.c_int64), ("n_units", ctypes.c_int64),
        ("n_routes", ctypes.c_int32), ("dtype", ctypes.c_int32),
        ("gate", ctypes.c_int32), ("stats_mode", ctypes.c_int32),
        ("sharpness", ctypes.c_float), ("act_threshold", ctypes.c_float),
        ("act_cutoff", ctypes.c_float), ("epsilon", ctypes.c_float),
        ("max_intensity", ctypes.c_float), ("dead_threshold", ctypes.c_float),
        ("scale", ctypes.c_float), ("chunk_size", ctypes.c_int32),
        ("flags", ctypes.c_uint32), ("reserved", ctypes.c_int32 * 3),
    ]


class SrwTensors(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("x", "h", "emb", "tau_offset", "read", "write")]


class SrwOutputs(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in (
        "out", "gate_sum", "den", "n_active", "pass_mask", "token_diag", "unit_diag", "gate")]


class SrwCotangents(ctypes.Structure):
    _fields_ = [("d_out", ctypes.c_void_p), ("out", ctypes.c_void_p),
                ("d_score_lb", ctypes.c_float), ("d_dead_penalty", ctypes.c_float),
                ("den", ctypes.c_void_p), ("unit_diag", ctypes.c_void_p)]


class SrwGrads(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in (
        "dx", "dh", "demb", "dtau_offset", "dread", "dwrite", "dscale")]


class SrwError(RuntimeError):
    """A non-OK status returned by libsrw_amd.so."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


class SrwLibraryError(RuntimeError):
    """libsrw_amd.so is missing or does not match this binding."""


_lib = None
_lock = threading.Lock()


def load_library() -> ctypes.CDLL:
    """Load (once) and return libsrw_amd.so; raise if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise SrwLibraryError(
                f"{LIB_PATH} is not built; run __graft_entry__.build() "
                "(make -C dawn-srw_amd/csrc) first")
        lib = ctypes.CDLL(LIB_PATH)
        lib.srw_abi_version.restype = ctypes.c_int32
        lib.srw_abi_version.argtypes = []
        lib.srw_status_string.restype = ctypes.c_char_p
        lib.srw_status_string.argtypes = [ctypes.c_int]
        lib.srw_desc_init.restype = ctypes.c_int
        lib.srw_desc_init.argtypes = [ctypes.POINTER(SrwDesc)]
        lib.srw_workspace_size.restype = ctypes.c_int
        lib.srw_workspace_size.argtypes = [ctypes.POINTER(SrwDesc), ctypes.POINTER(ctypes.c_size_t)]
        lib.srw_forward.restype = ctypes.c_int
        lib.srw_forward.argtypes = [
            ctypes.POINTER(SrwDesc), ctypes.POINTER(SrwTensors), ctypes.POINTER(SrwOutputs),
            ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
        lib.srw_forward_noalloc.restype = ctypes.c_int
        lib.srw_forward_noalloc.argtypes = [
            ctypes.POINTER(SrwDesc), ctypes.POINTER(SrwTensors), ctypes.POINTER(SrwOutputs),
            ctypes.c_void_p]
        lib.srw_workspace_size_batch.restype = ctypes.c_int
        lib.srw_workspace_size_batch.argtypes = [ctypes.c_int32, ctypes.POINTER(SrwDesc),
                                                 ctypes.POINTER(ctypes.c_size_t)]
        lib.srw_forward_batch.restype = ctypes.c_int
        lib.srw_forward_batch.argtypes = [
            ctypes.c_int32, ctypes.POINTER(SrwDesc), ctypes.POINTER(SrwTensors), ctypes.POINTER(SrwOutputs),
            ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
        lib.srw_last_path.restype = ctypes.c_char_p
        lib.srw_last_path.argtypes = []
        lib.srw_set_kernel_events.restype = ctypes.c_int
        lib.srw_set_kernel_events.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        lib.srw_backward_workspace_size.restype = ctypes.c_int
        lib.srw_backward_workspace_size.argtypes = [ctypes.POINTER(SrwDesc), ctypes.POINTER(ctypes.c_size_t)]
        lib.srw_backward.restype = ctypes.c_int
        lib.srw_backward.argtypes = [
            ctypes.POINTER(SrwDesc), ctypes.POINTER(SrwTensors), ctypes.POINTER(SrwCotangents),
            ctypes.POINTER(SrwGrads), ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
        got = lib.srw_abi_version()
        if got != ABI_VERSION:
            raise SrwLibraryError(f"libsrw_amd.so ABI {got} != binding ABI {ABI_VERSION}")
        _lib = lib
    return _lib


def check(status: int) -> None:
    if status != SRW_OK:
        msg = load_library().srw_status_string(status).decode()
        raise SrwError(status, msg)


def desc_init() -> SrwDesc:
    d = SrwDesc()
    check(load_library().srw_desc_init(ctypes.byref(d)))
    return d


def workspace_size(desc: SrwDesc) -> int:
    n = ctypes.c_size_t(0)
    check(load_library().srw_workspace_size(ctypes.byref(desc), ctypes.byref(n)))
    return int(n.value)


def workspace_size_batch(descs) -> int:
    """srw_workspace_size_batch over a ctypes array of SrwDesc."""
    n = ctypes.c_size_t(0)
    check(load_library().srw_workspace_size_batch(len(descs), descs, ctypes.byref(n)))
    return int(n.value)


def backward_workspace_size(desc: SrwDesc) -> int:
    n = ctypes.c_size_t(0)
    check(load_library().srw_backward_workspace_size(ctypes.byref(desc), ctypes.byref(n)))
    return int(n.value)


def last_path() -> str:
    return load_library().srw_last_path().decode()


def set_kernel_events(start, stop) -> None:
    """Install (or, with None, None, clear) the hipEvent_t handles that
    srw_forward records around its dominant kernel on this thread."""
    check(load_library().srw_set_kernel_events(
        ctypes.c_void_p(start or 0), ctypes.c_void_p(stop or 0)))
