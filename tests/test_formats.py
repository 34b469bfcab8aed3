"""The reference's on-disk formats, CPU only: pretokenized uint16 ``.bin``
token files (utils/data_jax.py:48-282) and ``.flax`` msgpack checkpoints
(scripts/train_jax.py:1096-1154).

The reference ships neither kind of file, and flax (the checkpoint format's
owner) is not in this image, so the checkpoint reader is pinned by bytes
written here directly with msgpack in flax's published layout (nested maps,
arrays as extension type 1 holding (shape, dtype name, bytes), numpy scalars
as type 3, oversized arrays as chunk maps) -- independent of this package's
writer -- and by a round trip through the writer; bit-level agreement with
files flax itself wrote is parity unpinned.
"""

from __future__ import annotations

import json

import msgpack
import numpy as np
import pytest
import torch


def _ext_array(a: np.ndarray, name: str | None = None):
    return msgpack.ExtType(1, msgpack.packb((list(a.shape), name or a.dtype.name, a.tobytes()), use_bin_type=True))


def test_bin_dataset_rows_and_batches(pkg, tmp_path):
    toks = np.arange(1000, dtype=np.uint16) * 7
    path = tmp_path / "c4_val.bin"
    toks.tofile(path)
    ds = pkg.data.BinDataset(str(path), seq_len=64)
    assert len(ds) == 1000 // 64                              # the tail of 40 tokens is dropped
    b = ds.get_batch(3, 4)
    assert b.dtype == np.int32 and b.shape == (4, 64)
    assert np.array_equal(b, toks[3 * 64:7 * 64].reshape(4, 64).astype(np.int32))
    assert ds.get_batch(14, 8).shape == (1, 64)               # short last batch
    assert ds.get_batch(15, 8) is None
    assert len(pkg.data.BinDataset(str(path), seq_len=64, max_sequences=5)) == 5
    with pytest.raises(ValueError, match="no full row"):
        pkg.data.BinDataset(str(path), seq_len=4096)


def test_sharded_dataset_spans_shards(pkg, tmp_path):
    rows = []
    shards = []
    for i, n in enumerate((5, 3, 4)):
        t = (np.arange(n * 16, dtype=np.uint16) + 1000 * i)
        t.tofile(tmp_path / f"shard_{i}.bin")
        rows.append(t.reshape(n, 16))
        shards.append({"path": f"shard_{i}.bin", "sequences": n, "tokens": n * 16})
    (tmp_path / "train_meta.json").write_text(json.dumps({"shards": shards, "vocab_size": 32000}))
    ds = pkg.data.ShardedBinDataset(str(tmp_path / "train_meta.json"), seq_len=16)
    allrows = np.concatenate(rows).astype(np.int32)
    assert len(ds) == 12 and ds.vocab_size == 32000
    assert np.array_equal(ds.get_batch(3, 6), allrows[3:9])   # spans shards 0, 1, 2
    assert np.array_equal(ds.get_batch(10, 5), allrows[10:12])
    assert ds.get_batch(12, 1) is None
    shards[1]["sequences"] = 9                                  # the file holds 3
    (tmp_path / "bad_meta.json").write_text(json.dumps({"shards": shards}))
    with pytest.raises(ValueError, match="fewer rows"):
        pkg.data.ShardedBinDataset(str(tmp_path / "bad_meta.json"), seq_len=16).get_batch(5, 6)


def test_flax_layout_is_read(pkg, tmp_path):
    """Bytes in flax's layout, written here with msgpack alone."""
    g = np.random.default_rng(0)
    emb = g.standard_normal((1, 40, 16)).astype(np.float32)   # device-replicated: leading axis 1
    scale = np.array([19.5959], dtype=np.float32)
    w_bf = (g.standard_normal((8, 4)).astype(np.float32))
    bf_bits = (torch.from_numpy(w_bf).to(torch.bfloat16).view(torch.uint16).numpy())
    big = g.standard_normal(10).astype(np.float32)
    tree = {
        "params": {"neuron_pool": {"know_emb": _ext_array(emb), "know_scale": _ext_array(scale)},
                   "block_0": {"attn": {"expand_O": {"kernel": _ext_array(bf_bits, "bfloat16")}}},
                   # flax's _chunk: shape and pieces both as maps keyed '0', '1', ... (_tuple_to_dict)
                   "chunked": {"__msgpack_chunked_array__": True, "shape": {"0": 2, "1": 5},
                               "chunks": {"0": _ext_array(big[:6]), "1": _ext_array(big[6:])}},
                   # a shape stored as a list is read as well
                   "chunked_list": {"__msgpack_chunked_array__": True, "shape": [5, 2],
                                    "chunks": {"0": _ext_array(big[:4]), "1": _ext_array(big[4:])}}},
        "opt_state": {"0": {"count": msgpack.ExtType(3, msgpack.packb(([], "int32", np.int32(7).tobytes())))},
                      "1": {}},
        "epoch": 2, "step": 12345, "best_val_loss": 3.25, "config": {"d_model": 16, "n_know": 40},
    }
    path = tmp_path / "best_model.flax"
    path.write_bytes(msgpack.packb(tree, use_bin_type=True))
    ckpt = pkg.checkpoint.load_checkpoint(str(path))
    assert ckpt["step"] == 12345 and ckpt["epoch"] == 2 and ckpt["best_val_loss"] == 3.25
    assert int(ckpt["opt_state"]["0"]["count"]) == 7
    p = ckpt["params"]
    assert torch.equal(p["neuron_pool"]["know_emb"], torch.from_numpy(emb))
    assert p["block_0"]["attn"]["expand_O"]["kernel"].dtype == torch.bfloat16
    assert torch.equal(p["block_0"]["attn"]["expand_O"]["kernel"].float(),
                       torch.from_numpy(w_bf).to(torch.bfloat16).float())
    assert torch.equal(p["chunked"], torch.from_numpy(big.reshape(2, 5)))
    assert torch.equal(p["chunked_list"], torch.from_numpy(big.reshape(5, 2)))
    params = pkg.checkpoint.load_params(str(path))
    assert params["neuron_pool"]["know_emb"].shape == (40, 16)      # leading replica axis dropped
    assert params["neuron_pool"]["know_scale"].shape == (1,)        # 1-d arrays keep it
    assert params["block_0"]["attn"]["expand_O"]["kernel"].dtype == torch.float32
    cfg = pkg.checkpoint.config_from_checkpoint(ckpt, n_layers=1)
    assert (cfg.d_model, cfg.n_know, cfg.n_layers) == (16, 40, 1)


def test_flax_reader_rejects_what_is_not_data(pkg, tmp_path):
    path = tmp_path / "x.flax"
    path.write_bytes(msgpack.packb({"params": msgpack.ExtType(42, b"\x00")}, use_bin_type=True))
    with pytest.raises(ValueError, match="extension type 42"):
        pkg.checkpoint.load_checkpoint(str(path))
    path.write_bytes(msgpack.packb([1, 2, 3]))
    with pytest.raises(ValueError, match="not a checkpoint"):
        pkg.checkpoint.load_checkpoint(str(path))
    path.write_bytes(msgpack.packb({"params": msgpack.ExtType(1, msgpack.packb(([2], "object", b"")))}))
    with pytest.raises(ValueError, match="object"):
        pkg.checkpoint.load_checkpoint(str(path))


def test_model_params_round_trip(pkg, tmp_path):
    cfg = pkg.DawnConfig(vocab_size=50, d_model=32, n_layers=2, n_heads=2, max_seq_len=16, d_route=16,
                         n_qk=40, n_v=50, n_know=120)
    params = pkg.init_params(cfg, seed=1)
    path = tmp_path / "checkpoint_epoch1.flax"
    pkg.checkpoint.save_checkpoint(str(path), params, opt_state=({"mu": params["norm"]["scale"]}, {}),
                                   epoch=1, step=99, config={"vocab_size": 50, "d_model": 32, "n_layers": 2})
    back = pkg.checkpoint.load_params(str(path))

    def flat(t, pre=""):
        if isinstance(t, dict):
            out = {}
            for k, v in t.items():
                out.update(flat(v, f"{pre}/{k}"))
            return out
        return {pre: t}

    a, b = flat(params), flat(back)
    assert a.keys() == b.keys()
    for k in a:
        assert torch.equal(a[k], b[k]), k
    ckpt = pkg.checkpoint.load_checkpoint(str(path))
    assert ckpt["step"] == 99 and torch.equal(ckpt["opt_state"]["0"]["mu"], params["norm"]["scale"])
    assert pkg.checkpoint.config_from_checkpoint(ckpt).vocab_size == 50


def test_chunked_array_round_trip(pkg, tmp_path, monkeypatch):
    """An array above the chunk limit is written as flax's _chunk writes it
    (shape and pieces as maps keyed '0', '1', ...) and read back whole."""
    monkeypatch.setattr(pkg.checkpoint, "_MAX_CHUNK", 64)       # bytes: forces several pieces
    big = torch.arange(3 * 7 * 5, dtype=torch.float32).reshape(3, 7, 5)
    path = tmp_path / "chunked.flax"
    pkg.checkpoint.save_checkpoint(str(path), {"pool": {"w": big}})
    raw = msgpack.unpackb(path.read_bytes(), raw=False, strict_map_key=False)
    stored = raw["params"]["pool"]["w"]
    assert stored["__msgpack_chunked_array__"] is True
    assert stored["shape"] == {"0": 3, "1": 7, "2": 5}
    assert len(stored["chunks"]) > 1 and set(stored["chunks"]) == {str(i) for i in range(len(stored["chunks"]))}
    back = pkg.checkpoint.load_checkpoint(str(path))["params"]["pool"]["w"]
    assert torch.equal(back, big)
