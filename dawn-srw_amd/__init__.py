"""dawn-srw_amd: MI355X-native Select-Read-Write (SRW) unit-pool layer.

The hot path of madst0614/DAWN-SRW (the fused gate + SRW function of
models/dawn_spatial_v41_exp.py:352-909 and its inference twin :1713-1738)
rebuilt as hand-written gfx950 HIP kernels behind a C ABI
(include/srw_amd.h, lib/libsrw_amd.so).  This package is the Python host
side: a ctypes binding, a tensor-level wrapper and a drop-in mirror of the
reference factories.

The directory name is not a Python identifier; load the package with
``__graft_entry__.load_package()``, which registers it as ``dawn_srw_amd``.
"""

from ._capi import SrwError, SrwLibraryError, load_library  # noqa: F401
from .layer import GateConfig, SrwBackwardPlan, SrwBatchPlan, SrwPlan, srw_backward, srw_forward  # noqa: F401
from .srw import (chunk_plan, make_sharded_srw, make_sharded_srw_paired, make_sharded_srw_v401,  # noqa: F401
                  make_sharded_srw_paired_v401, srw_inference, srw_inference_with_gates)
from . import checkpoint, data, inputs, model  # noqa: F401
from .model import DawnConfig, DawnModel, init_params  # noqa: F401

__all__ = ["SrwError", "SrwLibraryError", "load_library", "GateConfig",
           "SrwPlan", "SrwBatchPlan", "SrwBackwardPlan", "srw_forward", "srw_backward", "chunk_plan",
           "make_sharded_srw", "make_sharded_srw_paired", "make_sharded_srw_v401",
           "make_sharded_srw_paired_v401", "srw_inference", "srw_inference_with_gates",
           "inputs", "model", "checkpoint", "data", "DawnConfig", "DawnModel", "init_params"]
