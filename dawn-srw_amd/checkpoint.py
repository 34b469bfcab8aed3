"""Reading and writing the reference's ``.flax`` checkpoints.

The reference saves ``flax.serialization.to_bytes(ckpt)`` of the dict
``{'params', 'opt_state', 'epoch', 'step', 'step_in_epoch',
'steps_per_epoch', 'best_val_loss', 'config', 'training_config'}``
(scripts/train_jax.py:1096-1116) and restores it with ``from_bytes``
(:1135-1154).  That byte format is flax's msgpack serialization (flax is a
third-party dependency, ``flax>=0.7.0`` in requirements_tpu.txt:3, not in
this image), restated here from its published layout:

* the pytree as nested msgpack maps with string keys (sequences become maps
  keyed ``'0'``, ``'1'``, ...);
* every array as msgpack extension type 1 whose payload is the msgpack
  triple ``(shape, dtype name, C-order bytes)``; numpy scalars as extension
  type 3 with the same payload; Python complex numbers as type 2, a pair;
* arrays above flax's chunk size as a map ``{'__msgpack_chunked_array__':
  True, 'shape': ..., 'chunks': {'0': flat piece, ...}}``.

Decoding is data only (msgpack maps, numbers, strings and byte payloads):
nothing in the file is executed.  ``bfloat16`` arrays (dtype name
``'bfloat16'``, which numpy does not know) load as ``torch.bfloat16``.
``load_params`` also applies the reference's ``_squeeze_params``
(models/dawn_spatial_v41_exp.py:1700-1710): a leading axis of size 1 (device-
replicated checkpoints) is dropped.
"""

from __future__ import annotations

import numpy as np
import torch

try:
    import msgpack
except ImportError:  # pragma: no cover - the image ships msgpack
    msgpack = None

__all__ = ["load_checkpoint", "load_params", "save_checkpoint", "config_from_checkpoint"]

_EXT_NDARRAY, _EXT_COMPLEX, _EXT_NPSCALAR = 1, 2, 3
_CHUNKED = "__msgpack_chunked_array__"
_MAX_CHUNK = (1 << 30) - (1 << 20)  # bytes per chunk when writing large arrays


def _need_msgpack():
    if msgpack is None:
        raise ImportError("reading .flax checkpoints needs the msgpack package")


def _array_from_payload(data: bytes):
    shape, dtype_name, buf = msgpack.unpackb(data, raw=False)
    if isinstance(dtype_name, bytes):
        dtype_name = dtype_name.decode()
    shape = tuple(int(s) for s in shape)
    if dtype_name == "bfloat16":
        raw = np.frombuffer(buf, dtype=np.uint16).reshape(shape)
        return torch.from_numpy(raw.copy()).view(torch.bfloat16)
    dt = np.dtype(dtype_name)
    if dt.hasobject:
        raise ValueError(f"array of object dtype {dtype_name!r} in checkpoint")
    return torch.from_numpy(np.frombuffer(buf, dtype=dt).reshape(shape).copy())


def _ext_hook(code, data):
    if code == _EXT_NDARRAY:
        return _array_from_payload(data)
    if code == _EXT_NPSCALAR:
        return _array_from_payload(data).reshape(())
    if code == _EXT_COMPLEX:
        re, im = msgpack.unpackb(data, raw=False)
        return complex(re, im)
    raise ValueError(f"unknown msgpack extension type {code} in checkpoint")


def _dict_to_list(d):
    """flax's _dict_to_tuple: a map keyed '0', '1', ... (how flax's _chunk
    stores both the shape and the pieces of a chunked array) as a list; a
    list is taken as it is."""
    if isinstance(d, dict):
        return [d[str(i)] for i in range(len(d))]
    return list(d)


def _unchunk(tree):
    if isinstance(tree, dict):
        if tree.get(_CHUNKED) is True:
            shape = tuple(int(s) for s in _dict_to_list(tree["shape"]))
            pieces = _dict_to_list(tree["chunks"])
            flat = torch.cat([p.reshape(-1) for p in pieces])
            return flat.reshape(shape)
        return {k: _unchunk(v) for k, v in tree.items()}
    return tree


def load_checkpoint(path: str) -> dict:
    """The checkpoint dict of a ``.flax`` file (local path), arrays as CPU
    torch tensors in their stored dtype."""
    _need_msgpack()
    with open(path, "rb") as f:
        data = f.read()
    tree = msgpack.unpackb(data, ext_hook=_ext_hook, raw=False, strict_map_key=False)
    if not isinstance(tree, dict):
        raise ValueError(f"{path}: not a checkpoint (top level is {type(tree).__name__})")
    return _unchunk(tree)


def _squeeze_leading(t):
    return t[0] if isinstance(t, torch.Tensor) and t.dim() >= 2 and t.shape[0] == 1 else t


def _tree_map(fn, tree):
    if isinstance(tree, dict):
        return {k: _tree_map(fn, v) for k, v in tree.items()}
    return fn(tree)


def load_params(path: str, dtype: torch.dtype = torch.float32) -> dict:
    """The ``params`` tree of a ``.flax`` checkpoint as float tensors (for
    :class:`DawnModel`), a leading replica axis of size 1 dropped
    (v41:1700-1710: arrays of two or more dimensions; the (1,)-shaped pool
    scales stay as they are)."""
    ckpt = load_checkpoint(path)
    if "params" not in ckpt:
        raise KeyError(f"{path}: checkpoint has no 'params' entry")

    def conv(t):
        if not isinstance(t, torch.Tensor):
            return t
        return _squeeze_leading(t).to(dtype)

    return _tree_map(conv, ckpt["params"])


def config_from_checkpoint(ckpt: dict, **overrides):
    """A :class:`DawnConfig` from the checkpoint's ``config`` entry (the
    model_config the reference stores), fields it does not hold at their
    defaults."""
    from .model import DawnConfig
    import dataclasses
    names = {f.name for f in dataclasses.fields(DawnConfig)}
    cfg = ckpt.get("config") or {}
    kw = {k: (int(v) if isinstance(v, (int, np.integer)) else v) for k, v in cfg.items() if k in names}
    kw.update(overrides)
    return DawnConfig(**kw)


# -- writing -----------------------------------------------------------------
def _array_payload(t) -> bytes:
    if isinstance(t, torch.Tensor):
        t = t.detach().cpu().contiguous()
        if t.dtype == torch.bfloat16:
            return msgpack.packb((list(t.shape), "bfloat16", t.view(torch.uint16).numpy().tobytes()),
                                 use_bin_type=True)
        t = t.numpy()
    a = np.ascontiguousarray(t)
    return msgpack.packb((list(a.shape), a.dtype.name, a.tobytes()), use_bin_type=True)


def _to_state(tree):
    if isinstance(tree, dict):
        return {str(k): _to_state(v) for k, v in tree.items()}
    if isinstance(tree, (list, tuple)):
        return {str(i): _to_state(v) for i, v in enumerate(tree)}
    if isinstance(tree, torch.Tensor) or isinstance(tree, np.ndarray):
        nbytes = tree.numel() * tree.element_size() if isinstance(tree, torch.Tensor) else tree.nbytes
        if nbytes > _MAX_CHUNK:
            flat = tree.reshape(-1)
            per = max(1, _MAX_CHUNK // (nbytes // max(1, flat.shape[0])))
            chunks = {str(i): flat[j:j + per] for i, j in enumerate(range(0, flat.shape[0], per))}
            shape = {str(i): int(n) for i, n in enumerate(tree.shape)}  # flax's _tuple_to_dict
            return {_CHUNKED: True, "shape": shape, "chunks": chunks}
    return tree


def _default(x):
    if isinstance(x, (torch.Tensor, np.ndarray)):
        return msgpack.ExtType(_EXT_NDARRAY, _array_payload(x))
    if isinstance(x, np.generic):
        return msgpack.ExtType(_EXT_NPSCALAR, _array_payload(np.asarray(x)))
    if isinstance(x, complex):
        return msgpack.ExtType(_EXT_COMPLEX, msgpack.packb((x.real, x.imag)))
    raise TypeError(f"cannot serialise {type(x).__name__}")


def save_checkpoint(path: str, params: dict, *, opt_state=None, epoch: int = 0, step: int = 0,
                    best_val_loss: float = float("inf"), config: dict | None = None,
                    step_in_epoch: int = 0, steps_per_epoch: int = 0,
                    training_config: dict | None = None) -> None:
    """Write a checkpoint in the layout the reference's save_checkpoint
    produces (scripts/train_jax.py:1096-1132)."""
    _need_msgpack()
    ckpt = {"params": params, "opt_state": opt_state if opt_state is not None else {}, "epoch": epoch,
            "step": step, "step_in_epoch": step_in_epoch, "steps_per_epoch": steps_per_epoch,
            "best_val_loss": best_val_loss, "config": config or {}, "training_config": training_config or {}}
    data = msgpack.packb(_to_state(ckpt), default=_default, use_bin_type=True, strict_types=False)
    with open(path, "wb") as f:
        f.write(data)
