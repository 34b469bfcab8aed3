"""Restatement of the DAWN-SRW v4.1 model around the SRW layer (CPU).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.  Never imported by
the product path.

Follows models/dawn_spatial_v41_exp.py line by line, with dropout off
(deterministic=True):

* ``forward``      -- ``DAWN.__call__`` (:1285-1672) returning the logits
  (``token_emb.attend``, :1670), scan body ``_attn_forward`` (:983-1139) and
  ``_know_forward`` (:1142-1205); the SRW calls are the restated
  ``fused_gate_srw_paired`` (QK) and ``fused_gate_srw`` (V, Know) in bf16
  emulation with the training chunk plan;
* ``prefill`` / ``decode_step`` -- the KV-cache inference API (:1831-1957,
  ``_attn_forward_cached`` :1772-1817, ``_know_forward_inference``
  :1820-1828), whose SRW layer is ``_srw_inference`` (centred statistics),
  here at bf16 SRW inputs (``srw_dtype``) or float32; Q and K are two
  separate calls, as the reference makes them (:1788-1793).

Glue (embeddings, LayerNorm, router, attention, expand_O, logits) in
float32 with explicit formulas: the attention is the reference's einsum /
causal mask with finfo.min / softmax (:1063-1071), the LayerNorm its
mean / biased variance / eps 1e-6 (:321-324).  Pinned in
tests/test_model_oracle.py against library routines (torch layer_norm,
scaled_dot_product_attention), a closed form (expand_O = 0 and pool scales 0
reduce the model to LN(embedding) . E^T), causality and the KV-cache
identity (prefill + one decode step == prefill of the longer prompt).
"""

from __future__ import annotations

import torch

from oracle import srw_ref

F32 = torch.float32
BF16 = torch.bfloat16

__all__ = ["layer_norm", "causal_attention", "forward", "prefill", "decode_step"]


def layer_norm(x, scale, bias, eps=1e-6):
    """_layer_norm (v41:321-324)."""
    mean = x.mean(dim=-1, keepdim=True)
    var = torch.square(x - mean).mean(dim=-1, keepdim=True)
    return (x - mean) / torch.sqrt(var + eps) * scale + bias


def causal_attention(Q, K, V):
    """Q, K, V [B, H, S, dh] -> [B, H, S, dh] (v41:1063-1071): scores / sqrt(dh),
    entries above the diagonal set to finfo.min, softmax over keys."""
    S, dh = Q.shape[-2], Q.shape[-1]
    scale = torch.sqrt(torch.tensor(float(dh), dtype=Q.dtype))
    scores = torch.einsum("bhsd,bhtd->bhst", Q, K) / scale
    causal = torch.tril(torch.ones(S, S, dtype=torch.bool))
    scores = torch.where(causal, scores, torch.tensor(torch.finfo(scores.dtype).min, dtype=scores.dtype))
    w = torch.softmax(scores, dim=-1)
    return torch.einsum("bhst,bhtd->bhsd", w, V)


def _heads(t, n_heads):
    B, S, D = t.shape
    return t.reshape(B, S, n_heads, D // n_heads).transpose(1, 2)


def _merge(t):
    B, H, S, dh = t.shape
    return t.transpose(1, 2).reshape(B, S, H * dh)


def _dense(x, prm):
    return x @ prm["kernel"] + prm["bias"]


def _route_blocks(h_all, dr):
    """h_Q, h_K, h_V: the router output split in three along the last axis
    (jnp.split(h_all, 3, axis=-1), v41:1019)."""
    return h_all[..., :dr], h_all[..., dr:2 * dr], h_all[..., 2 * dr:]


def _tau_columns(tau_all):
    """tau_offset of Q, K and V: columns 0, 1, 2 of the tau router (v41:1036, :1053)."""
    return tau_all[..., 0:1], tau_all[..., 1:2], tau_all[..., 2:3]


def _qk_scaled(QK, qk_scale):
    """Q and K from the paired call's two routes, both times qk_scale (v41:1044-1045)."""
    return QK[:, :, 0, :] * qk_scale, QK[:, :, 1, :] * qk_scale


def forward(params, cfg, input_ids, *, max_chunk_size=None):
    """logits [B, S, vocab] of DAWN.__call__(input_ids, deterministic=True)."""
    chunk = cfg.max_chunk_size if max_chunk_size is None else max_chunk_size
    B, S = input_ids.shape
    dr, H = cfg.d_route, cfg.n_heads
    pool, rt = params["neuron_pool"], params["router"]
    x = params["token_emb"]["embedding"][input_ids] + params["pos_emb"]["embedding"][:S][None]  # :1291-1292
    for i in range(cfg.n_layers):
        bp = params[f"block_{i}"]
        normed = layer_norm(x, bp["norm1"]["scale"], bp["norm1"]["bias"])          # :1412-1413
        h_Q, h_K, h_V = _route_blocks(_dense(normed, rt["proj_attn"]), dr)       # :1018-1019
        t_Q, t_K, t_V = _tau_columns(_dense(normed, rt["tau_attn"]))             # :1022
        h_QK = torch.stack([h_Q, h_K], dim=2)                                    # :1035
        tau_QK = torch.stack([t_Q, t_K], dim=2)                                  # :1036
        QK = srw_ref.fused_gate_srw_paired(normed, h_QK, pool["qk_emb"], tau_QK, pool["qk_read"],
                                           pool["qk_write"], max_chunk_size=chunk)[0]
        Q, K = _qk_scaled(QK, pool["qk_scale"])                                  # :1044-1045
        V = srw_ref.fused_gate_srw(normed, h_V, pool["v_emb"], t_V, pool["v_read"],
                                   pool["v_write"], max_chunk_size=chunk)[0] * pool["v_scale"]  # :1046-1053
        a = _merge(causal_attention(_heads(Q, H), _heads(K, H), _heads(V, H)))   # :1056-1081
        x = x + a @ bp["attn"]["expand_O"]["kernel"]                             # :1082, :1438
        normed = layer_norm(x, bp["norm2"]["scale"], bp["norm2"]["bias"])        # :1440-1441
        h = _dense(normed, rt["proj_know"])                                      # :1151
        tau = _dense(normed, rt["tau_know"])                                     # :1156
        know = srw_ref.fused_gate_srw(normed, h, pool["know_emb"], tau, pool["know_read"],
                                      pool["know_write"], max_chunk_size=chunk)[0]
        x = x + know * pool["know_scale"]                                        # :1175, :1457
    x = layer_norm(x, params["norm"]["scale"], params["norm"]["bias"])           # :1542
    return x @ params["token_emb"]["embedding"].T                                # :1670


def _srw_inf(x, h, emb, tau, read, write, srw_dtype):
    """_srw_inference (v41:1713-1738) with the SRW inputs in ``srw_dtype``
    (bf16: the bf16 dots of the oracle, f32 accumulation points), out f32."""
    c = lambda t: t.to(srw_dtype)  # noqa: E731
    return srw_ref.srw_inference(c(x), c(h), c(emb), tau.to(F32), c(read), c(write))


def _attn_qkv(normed, params, cfg, srw_dtype):
    pool, rt = params["neuron_pool"], params["router"]
    dr = cfg.d_route
    h_Q, h_K, h_V = _route_blocks(_dense(normed, rt["proj_attn"]), dr)           # :1784 / :1866
    t_Q, t_K, t_V = _tau_columns(_dense(normed, rt["tau_attn"]))
    Q = _srw_inf(normed, h_Q, pool["qk_emb"], t_Q, pool["qk_read"], pool["qk_write"], srw_dtype)
    K = _srw_inf(normed, h_K, pool["qk_emb"], t_K, pool["qk_read"], pool["qk_write"], srw_dtype)
    V = _srw_inf(normed, h_V, pool["v_emb"], t_V, pool["v_read"], pool["v_write"], srw_dtype)
    return Q * pool["qk_scale"], K * pool["qk_scale"], V * pool["v_scale"]      # :1794-1799, :1876-1880


def _know_inf(normed, params, srw_dtype):
    pool, rt = params["neuron_pool"], params["router"]
    h = _dense(normed, rt["proj_know"])                                          # :1824-1825
    tau = _dense(normed, rt["tau_know"])
    out = _srw_inf(normed, h, pool["know_emb"], tau, pool["know_read"], pool["know_write"], srw_dtype)
    return out * pool["know_scale"]                                              # :1828


def prefill(params, cfg, input_ids, *, srw_dtype=BF16):
    """(logits [B, S, vocab], cache_K, cache_V [L, B, H, max_seq, dh], S)
    of the reference's prefill (v41:1831-1910)."""
    B, S = input_ids.shape
    D, H, L = cfg.d_model, cfg.n_heads, cfg.n_layers
    dh = D // H
    cK = torch.zeros(L, B, H, cfg.max_seq_len, dh)
    cV = torch.zeros_like(cK)
    x = params["token_emb"]["embedding"][input_ids] + params["pos_emb"]["embedding"][:S][None]  # :1847-1848
    for i in range(L):
        bp = params[f"block_{i}"]
        normed = layer_norm(x, bp["norm1"]["scale"], bp["norm1"]["bias"])
        Q, K, V = _attn_qkv(normed, params, cfg, srw_dtype)
        Qh, Kh, Vh = _heads(Q, H), _heads(K, H), _heads(V, H)
        cK[i, :, :, :S] = Kh                                                     # :1886-1887
        cV[i, :, :, :S] = Vh
        x = x + _merge(causal_attention(Qh, Kh, Vh)) @ bp["attn"]["expand_O"]["kernel"]  # :1889-1897
        normed = layer_norm(x, bp["norm2"]["scale"], bp["norm2"]["bias"])
        x = x + _know_inf(normed, params, srw_dtype)                             # :1899-1901
    x = layer_norm(x, params["norm"]["scale"], params["norm"]["bias"])
    return x @ params["token_emb"]["embedding"].T, cK, cV, S


def decode_step(params, cfg, token_id, cache_K, cache_V, cache_len, *, srw_dtype=BF16):
    """(logits [B, vocab], cache_K, cache_V, cache_len + 1) of the reference's
    decode_step (v41:1914-1957); returns updated copies of the caches."""
    cache_K, cache_V = cache_K.clone(), cache_V.clone()
    ids = token_id.reshape(-1, 1)
    B = ids.shape[0]
    D, H = cfg.d_model, cfg.n_heads
    dh = D // H
    x = params["token_emb"]["embedding"][ids] + params["pos_emb"]["embedding"][cache_len][None, None]  # :1925-1926
    for i in range(cfg.n_layers):
        bp = params[f"block_{i}"]
        normed = layer_norm(x, bp["norm1"]["scale"], bp["norm1"]["bias"])
        Q, K, V = _attn_qkv(normed, params, cfg, srw_dtype)                      # [B, 1, D]
        cache_K[i, :, :, cache_len] = K.reshape(B, H, dh)                        # :1804-1805
        cache_V[i, :, :, cache_len] = V.reshape(B, H, dh)
        q = Q.reshape(B, H, 1, dh)
        scale = torch.sqrt(torch.tensor(float(dh)))
        sc = torch.einsum("bhqd,bhkd->bhqk", q, cache_K[i]) / scale              # :1807-1808
        pos_mask = torch.arange(cache_K.shape[3]) < (cache_len + 1)              # :1809
        sc = torch.where(pos_mask[None, None, None, :], sc, torch.tensor(torch.finfo(sc.dtype).min))
        a = torch.einsum("bhqk,bhkd->bhqd", torch.softmax(sc, dim=-1), cache_V[i])
        x = x + a.transpose(1, 2).reshape(B, 1, D) @ bp["attn"]["expand_O"]["kernel"]  # :1816-1817
        normed = layer_norm(x, bp["norm2"]["scale"], bp["norm2"]["bias"])
        x = x + _know_inf(normed, params, srw_dtype)
    x = layer_norm(x, params["norm"]["scale"], params["norm"]["bias"])
    return (x @ params["token_emb"]["embedding"].T)[:, 0, :], cache_K, cache_V, cache_len + 1
