"""The DAWN-SRW v4.1 language model around the SRW layer (one GPU).

Reference: madst0614/DAWN-SRW, models/dawn_spatial_v41_exp.py --
``DAWN.__call__`` (:1285-1672, deterministic: dropout off), its scan body
``_attn_forward`` (:983-1139) and ``_know_forward`` (:1142-1205), and the
inference API ``prefill`` / ``decode_step`` (:1831-1957) with
``_attn_forward_cached`` (:1772-1817) and ``_know_forward_inference``
(:1820-1828).

Every SRW call (the QK pool with its Q and K routes paired over one x.R^T,
the V pool, the Know pool) runs in libsrw_amd.so's HIP kernels.  The glue --
embeddings, LayerNorm (eps 1e-6, :321-324), the router Dense layers, causal
softmax attention, expand_O, the tied lm_head -- is plain float32 PyTorch, as
the reference computes it in float32.  Parameters use the reference's Flax
tree names (``params['neuron_pool']['know_emb']``,
``params['router']['proj_attn']['kernel']``, ``params['block_3']['norm1']
['scale']`` ...), so a checkpoint's tree maps onto them one to one.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from .layer import GateConfig, SrwBatchPlan, SrwPlan
from .srw import chunk_plan

__all__ = ["DawnConfig", "init_params", "DawnModel"]

BF16 = torch.bfloat16
F32 = torch.float32


@dataclass(frozen=True)
class DawnConfig:
    """Model shape (DAWN field defaults, v41:1246-1261; the 40M pools of
    configs/...v4_1...yaml:36-39).  ``max_chunk_size`` is the N-chunk the
    training script gives make_sharded_srw (scripts/train_jax.py:2326)."""
    vocab_size: int = 30000
    d_model: int = 384
    n_layers: int = 12
    n_heads: int = 6
    max_seq_len: int = 512
    d_route: int = 128
    n_qk: int = 1580
    n_v: int = 2600
    n_know: int = 25200
    max_chunk_size: int = 12500


def _unit_rows(g, n, d):
    """unit_norm_init (v41:333-338): N(0, 1) rows divided by (norm + 1e-8)."""
    x = torch.randn(n, d, generator=g)
    return x / (x.norm(dim=-1, keepdim=True) + 1e-8)


def _lecun_normal(g, fan_in, fan_out):
    """Flax's default Dense kernel init: truncated normal (+-2 sigma) with
    variance 1 / fan_in after truncation."""
    std = math.sqrt(1.0 / fan_in) / 0.87962566103423978
    w = torch.empty(fan_in, fan_out)
    torch.nn.init.trunc_normal_(w, 0.0, 1.0, -2.0, 2.0, generator=g)
    return w * std


def init_params(cfg: DawnConfig, seed: int = 0) -> dict:
    """Random-init parameters of the architecture (CPU, float32), with the
    reference's initialisers: embeddings and expand_O N(0, 0.02^2)
    (scaled_normal, v41:327-330), unit-norm pool rows, pool scales sqrt(D)
    (:945-950), Dense kernels lecun-normal with zero bias, tau kernels zero
    with bias -0.5 (:970-975), LayerNorm scale 1 / bias 0."""
    g = torch.Generator().manual_seed(seed)
    D, dr = cfg.d_model, cfg.d_route
    p = {
        "token_emb": {"embedding": 0.02 * torch.randn(cfg.vocab_size, D, generator=g)},
        "pos_emb": {"embedding": 0.02 * torch.randn(cfg.max_seq_len, D, generator=g)},
        "neuron_pool": {},
        "router": {
            "proj_attn": {"kernel": _lecun_normal(g, D, 3 * dr), "bias": torch.zeros(3 * dr)},
            "proj_know": {"kernel": _lecun_normal(g, D, dr), "bias": torch.zeros(dr)},
            "tau_attn": {"kernel": torch.zeros(D, 3), "bias": torch.full((3,), -0.5)},
            "tau_know": {"kernel": torch.zeros(D, 1), "bias": torch.full((1,), -0.5)},
        },
        "norm": {"scale": torch.ones(D), "bias": torch.zeros(D)},
    }
    pool = p["neuron_pool"]
    for name, n in (("qk", cfg.n_qk), ("v", cfg.n_v), ("know", cfg.n_know)):
        pool[f"{name}_emb"] = _unit_rows(g, n, dr)
        pool[f"{name}_read"] = _unit_rows(g, n, D)
        pool[f"{name}_write"] = _unit_rows(g, n, D)
        pool[f"{name}_scale"] = torch.full((1,), math.sqrt(D))
    for i in range(cfg.n_layers):
        p[f"block_{i}"] = {
            "norm1": {"scale": torch.ones(D), "bias": torch.zeros(D)},
            "norm2": {"scale": torch.ones(D), "bias": torch.zeros(D)},
            "attn": {"expand_O": {"kernel": 0.02 * torch.randn(D, D, generator=g)}},
        }
    return p


def _tree_map(fn, tree):
    if isinstance(tree, dict):
        return {k: _tree_map(fn, v) for k, v in tree.items()}
    return fn(tree)


class _PoolCall:
    """One pool's SRW call at a fixed token count: an ``SrwPlan`` bound to
    input buffers that the model fills in place, so the workspace, the
    outputs and the C descriptors are built once per shape."""

    def __init__(self, T, D, dr, R, emb, read, write, stats, chunk, device):
        self.x = torch.empty(T, D, dtype=BF16, device=device)
        self.h = torch.empty(T, R, dr, dtype=BF16, device=device)
        self.tau = torch.empty(T, R, dtype=F32, device=device)
        self.plan = SrwPlan(self.x, self.h, emb, self.tau, read, write, stats=stats,
                            consts=GateConfig(), chunk_size=chunk, want_mask=False)
        self.launches = 0

    def __call__(self, x, h, tau):
        self.x.copy_(x)
        self.h.copy_(h)
        self.tau.copy_(tau)
        # the pools are shared by all layers: after the first launch the
        # workspace's packed W^T is current
        self.plan.launch(pool_cached=self.launches > 0)
        self.launches += 1
        return self.plan.out


class _BatchCall:
    """Several pools' calls on the same rows as one ``srw_forward_batch``
    (one launch per stage when all take the decode kernel; the results equal
    separate calls bit for bit).  ``plan`` is the batch plan."""

    def __init__(self, *calls):
        self.calls = calls
        self.plan = SrwBatchPlan([c.plan for c in calls])
        self.launches = 0

    def __call__(self, *args):
        for c, (x, h, tau) in zip(self.calls, args):
            c.x.copy_(x)
            c.h.copy_(h)
            c.tau.copy_(tau)
        self.plan.launch(pool_cached=self.launches > 0)
        self.launches += 1
        return [c.plan.out for c in self.calls]


class DawnModel:
    """Inference on one HIP device.

    ``forward(ids)`` is ``DAWN.__call__(ids, deterministic=True)['logits']``
    (v41:1294-1700): fused_gate_srw semantics -- bf16 SRW with one-pass
    statistics and the training chunk plan.  ``prefill`` / ``decode_step``
    are the reference's KV-cache inference API (v41:1836-1957), whose SRW
    layer is ``_srw_inference`` (two-pass centred statistics, unchunked); it
    runs here in bf16 on the matrix cores, Q and K as one paired call over
    one x.R^T (the reference computes x.R^T twice, :1788-1793); at decode
    sizes the QK and V calls of a layer are one ``srw_forward_batch``.
    """

    def __init__(self, params: dict, cfg: DawnConfig, device="cuda:0"):
        self.cfg = cfg
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("DawnModel runs on a HIP device")
        if cfg.d_model % cfg.n_heads != 0:
            raise ValueError(f"d_model ({cfg.d_model}) must be divisible by n_heads ({cfg.n_heads})")
        self.p = _tree_map(lambda t: t.to(self.device, F32).contiguous(), params)
        pool = self.p["neuron_pool"]
        # the bf16 casts the SRW layer applies to the pool (v41:423-430), once
        self.pool_bf = {k: v.to(BF16).contiguous() for k, v in pool.items() if not k.endswith("_scale")}
        self.scale = {k: pool[f"{k}_scale"] for k in ("qk", "v", "know")}
        self._calls = {}

    # -- pieces -------------------------------------------------------------
    def _pool(self, name, T, R, stats):
        key = (name, T, R, stats)
        c = self._calls.get(key)
        if c is None:
            cfg = self.cfg
            N = self.pool_bf[f"{name}_emb"].shape[0]
            chunk = chunk_plan(N, cfg.max_chunk_size)[1] if stats == "onepass" else 0
            c = _PoolCall(T, cfg.d_model, cfg.d_route, R, self.pool_bf[f"{name}_emb"],
                          self.pool_bf[f"{name}_read"], self.pool_bf[f"{name}_write"], stats, chunk,
                          self.device)
            self._calls[key] = c
        return c

    def _qkv_batch(self, T, stats):
        key = ("qk+v", T, 1, stats)
        b = self._calls.get(key)
        if b is None:
            b = _BatchCall(self._pool("qk", T, 2, stats), self._pool("v", T, 1, stats))
            self._calls[key] = b
        return b

    @staticmethod
    def _ln(x, prm):
        return F.layer_norm(x, (x.shape[-1],), prm["scale"], prm["bias"], eps=1e-6)  # v41:321-324

    @staticmethod
    def _dense(x, prm):
        return torch.addmm(prm["bias"], x, prm["kernel"])

    def _srw_qkv(self, normed, stats):
        """Q, K, V of one layer (v41:1018-1053): router, paired QK call, V call,
        the pool scales applied after den (outside the SRW function)."""
        cfg, rt = self.cfg, self.p["router"]
        T, dr = normed.shape[0], cfg.d_route
        h_all = self._dense(normed, rt["proj_attn"])                    # :1018
        tau_all = self._dense(normed, rt["tau_attn"])                   # :1022
        qk_args = (normed, h_all[:, :2 * dr].reshape(T, 2, dr), tau_all[:, :2])
        v_args = (normed, h_all[:, 2 * dr:].reshape(T, 1, dr), tau_all[:, 2:3])
        if 2 * T <= 128:
            # decode-sized: both calls in one srw_forward_batch
            qk, v = self._qkv_batch(T, stats)(qk_args, v_args)
        else:
            qk = self._pool("qk", T, 2, stats)(*qk_args)
            v = self._pool("v", T, 1, stats)(*v_args)
        q = qk[:, 0].float() * self.scale["qk"]                         # :1044-1045
        k = qk[:, 1].float() * self.scale["qk"]
        v = v[:, 0].float() * self.scale["v"]                           # :1053
        return q, k, v

    def _know(self, normed, stats):
        """_know_forward (v41:1142-1175) / _know_forward_inference (:1820-1828)."""
        rt = self.p["router"]
        T = normed.shape[0]
        h = self._dense(normed, rt["proj_know"])
        tau = self._dense(normed, rt["tau_know"])
        out = self._pool("know", T, 1, stats)(normed, h[:, None], tau)
        return out[:, 0].float() * self.scale["know"]                   # :1175

    def _heads(self, t, B, S):
        H = self.cfg.n_heads
        return t.reshape(B, S, H, -1).transpose(1, 2)

    def _embed(self, ids, pos0=0):
        S = ids.shape[1]
        return (self.p["token_emb"]["embedding"][ids]
                + self.p["pos_emb"]["embedding"][pos0:pos0 + S][None])

    def _check_ids(self, ids):
        if ids.dim() != 2:
            raise ValueError("input_ids must be [B, S]")
        if ids.shape[1] > self.cfg.max_seq_len:
            raise ValueError(f"Sequence length {ids.shape[1]} exceeds max_seq_len")  # v41:1288-1289
        return ids.to(self.device)

    # -- DAWN.__call__ ------------------------------------------------------
    @torch.no_grad()
    def forward(self, input_ids) -> torch.Tensor:
        """logits [B, S, vocab] float32 (v41:1285-1672, deterministic=True)."""
        ids = self._check_ids(input_ids)
        B, S = ids.shape
        D = self.cfg.d_model
        x = self._embed(ids).reshape(B * S, D)
        for i in range(self.cfg.n_layers):
            bp = self.p[f"block_{i}"]
            q, k, v = self._srw_qkv(self._ln(x, bp["norm1"]), "onepass")
            a = F.scaled_dot_product_attention(self._heads(q, B, S), self._heads(k, B, S),
                                               self._heads(v, B, S), is_causal=True)   # :1063-1071
            x = x + a.transpose(1, 2).reshape(B * S, D) @ bp["attn"]["expand_O"]["kernel"]
            x = x + self._know(self._ln(x, bp["norm2"]), "onepass")
        x = self._ln(x, self.p["norm"])
        return (x @ self.p["token_emb"]["embedding"].T).reshape(B, S, -1)  # token_emb.attend, :1670

    # -- inference API ------------------------------------------------------
    @torch.no_grad()
    def prefill(self, input_ids):
        """(logits [B, S, vocab], cache_K, cache_V [L, B, H, max_seq, d_head],
        cache_len) as the reference's prefill (v41:1831-1910)."""
        ids = self._check_ids(input_ids)
        cfg = self.cfg
        B, S = ids.shape
        D, H, L = cfg.d_model, cfg.n_heads, cfg.n_layers
        dh = D // H
        cK = torch.zeros(L, B, H, cfg.max_seq_len, dh, device=self.device)
        cV = torch.zeros_like(cK)
        x = self._embed(ids).reshape(B * S, D)
        for i in range(L):
            bp = self.p[f"block_{i}"]
            q, k, v = self._srw_qkv(self._ln(x, bp["norm1"]), "centered")
            qh, kh, vh = self._heads(q, B, S), self._heads(k, B, S), self._heads(v, B, S)
            cK[i, :, :, :S] = kh
            cV[i, :, :, :S] = vh
            a = F.scaled_dot_product_attention(qh, kh, vh, is_causal=True)
            x = x + a.transpose(1, 2).reshape(B * S, D) @ bp["attn"]["expand_O"]["kernel"]
            x = x + self._know(self._ln(x, bp["norm2"]), "centered")
        x = self._ln(x, self.p["norm"])
        return (x @ self.p["token_emb"]["embedding"].T).reshape(B, S, -1), cK, cV, S

    @torch.no_grad()
    def decode_step(self, token_id, cache_K, cache_V, cache_len: int):
        """One token per sequence with the KV cache (v41:1914-1957):
        (logits [B, vocab], cache_K, cache_V, cache_len + 1).  The caches are
        updated in place."""
        cfg = self.cfg
        if cache_len >= cfg.max_seq_len:
            raise ValueError("KV cache is full")
        ids = token_id.reshape(-1, 1).to(self.device)
        B = ids.shape[0]
        D, H = cfg.d_model, cfg.n_heads
        dh = D // H
        x = self._embed(ids, pos0=cache_len).reshape(B, D)
        scale = math.sqrt(dh)
        for i in range(cfg.n_layers):
            bp = self.p[f"block_{i}"]
            q, k, v = self._srw_qkv(self._ln(x, bp["norm1"]), "centered")   # :1784-1799
            cache_K[i, :, :, cache_len] = k.reshape(B, H, dh)                # :1804-1805
            cache_V[i, :, :, cache_len] = v.reshape(B, H, dh)
            Kc = cache_K[i, :, :, :cache_len + 1]                            # positions < len + 1
            Vc = cache_V[i, :, :, :cache_len + 1]
            sc = torch.matmul(q.reshape(B, H, 1, dh), Kc.transpose(-1, -2).contiguous()) / scale  # :1807-1813
            a = torch.matmul(torch.softmax(sc, dim=-1), Vc.contiguous())
            x = x + a.reshape(B, D) @ bp["attn"]["expand_O"]["kernel"]
            x = x + self._know(self._ln(x, bp["norm2"]), "centered")
        x = self._ln(x, self.p["norm"])
        return x @ self.p["token_emb"]["embedding"].T, cache_K, cache_V, cache_len + 1
