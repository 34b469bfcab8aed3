"""Pins for the oracle's model restatement (oracle/dawn_ref.py), CPU only.

The glue around the SRW layer is checked against library routines (torch's
layer_norm and scaled_dot_product_attention), a closed form (zero expand_O
and zero pool scales leave logits = LN(token + position embedding) . E^T),
causality, and the KV-cache identity of the reference's inference API
(prefill of S tokens + one decode step == prefill of S + 1 tokens).  The SRW
calls themselves are the oracle functions pinned in test_oracle_pins.py.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from oracle import dawn_ref

F64 = torch.float64


@pytest.fixture(scope="module")
def tiny(pkg):
    cfg = pkg.model.DawnConfig(vocab_size=50, d_model=32, n_layers=2, n_heads=2, max_seq_len=16,
                               d_route=16, n_qk=40, n_v=50, n_know=120, max_chunk_size=60)
    return cfg, pkg.model.init_params(cfg, seed=3)


def _ids(B, S, vocab, seed):
    return torch.randint(0, vocab, (B, S), generator=torch.Generator().manual_seed(seed))


def test_layer_norm_matches_library():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(5, 7, 48, generator=g, dtype=F64)
    s, b = torch.randn(48, generator=g, dtype=F64), torch.randn(48, generator=g, dtype=F64)
    want = F.layer_norm(x, (48,), s, b, eps=1e-6)
    assert torch.allclose(dawn_ref.layer_norm(x, s, b), want, rtol=0, atol=1e-12)


def test_attention_matches_library_causal_sdpa():
    g = torch.Generator().manual_seed(1)
    Q, K, V = (torch.randn(2, 3, 11, 8, generator=g, dtype=F64) for _ in range(3))
    want = F.scaled_dot_product_attention(Q, K, V, is_causal=True)
    assert torch.allclose(dawn_ref.causal_attention(Q, K, V), want, rtol=0, atol=1e-12)


def test_zero_blocks_reduce_to_embedding_logits(tiny):
    cfg, p = tiny
    p = {k: (dict(v) if isinstance(v, dict) else v) for k, v in p.items()}
    p["neuron_pool"] = dict(p["neuron_pool"], know_scale=torch.zeros(1))
    for i in range(cfg.n_layers):
        p[f"block_{i}"] = dict(p[f"block_{i}"], attn={"expand_O": {"kernel": torch.zeros(32, 32)}})
    ids = _ids(2, 9, cfg.vocab_size, 4)
    x = p["token_emb"]["embedding"][ids] + p["pos_emb"]["embedding"][:9][None]
    want = F.layer_norm(x, (32,), p["norm"]["scale"], p["norm"]["bias"], eps=1e-6) @ p["token_emb"]["embedding"].T
    assert torch.allclose(dawn_ref.forward(p, cfg, ids), want, rtol=0, atol=1e-5)
    assert torch.allclose(dawn_ref.prefill(p, cfg, ids)[0], want, rtol=0, atol=1e-5)


def _causal_check(fn, cfg, p):
    ids = _ids(2, 12, cfg.vocab_size, 5)
    alt = ids.clone()
    alt[:, 7:] = (alt[:, 7:] + 1) % cfg.vocab_size
    a, b = fn(p, cfg, ids), fn(p, cfg, alt)
    return (a[:, :7] - b[:, :7]).abs().max().item(), (a[:, 7:] - b[:, 7:]).abs().max().item()


def test_logits_are_causal(tiny):
    cfg, p = tiny
    for fn in (dawn_ref.forward, lambda p_, c_, i_: dawn_ref.prefill(p_, c_, i_)[0]):
        before, after = _causal_check(fn, cfg, p)
        assert before <= 1e-6 and after > 1e-3, (before, after)


def test_planted_non_causal_attention_is_caught(tiny, monkeypatch):
    """An attention without the mask fails the causality check."""
    cfg, p = tiny
    monkeypatch.setattr(dawn_ref, "causal_attention",
                        lambda Q, K, V: F.scaled_dot_product_attention(Q, K, V, is_causal=False))
    before, _ = _causal_check(dawn_ref.forward, cfg, p)
    assert before > 1e-4


@pytest.mark.parametrize("srw_dtype", [torch.bfloat16, torch.float32])
def test_prefill_then_decode_equals_longer_prefill(tiny, srw_dtype):
    cfg, p = tiny
    ids = _ids(3, 10, cfg.vocab_size, 6)
    logits9, cK, cV, n = dawn_ref.prefill(p, cfg, ids[:, :9], srw_dtype=srw_dtype)
    step, cK2, cV2, n2 = dawn_ref.decode_step(p, cfg, ids[:, 9], cK, cV, n, srw_dtype=srw_dtype)
    full, fK, fV, _ = dawn_ref.prefill(p, cfg, ids, srw_dtype=srw_dtype)
    assert n2 == 10
    assert torch.allclose(step, full[:, 9], rtol=1e-4, atol=1e-5)
    assert torch.allclose(logits9, full[:, :9], rtol=1e-4, atol=1e-5)
    assert torch.allclose(cK2[:, :, :, :10], fK[:, :, :, :10], rtol=1e-4, atol=1e-6)
    assert torch.allclose(cV2[:, :, :, :10], fV[:, :, :, :10], rtol=1e-4, atol=1e-6)
    assert torch.count_nonzero(cK2[:, :, :, 10:]) == 0


# ---------------------------------------------------------------- router split, tau columns, scales

def _attn_params(cfg, p, seed):
    """One layer, the Know branch off (know_scale 0), distinct tau routers for
    Q, K and V (kernel and bias), so that the attention half of the block is
    the whole residual update."""
    g = torch.Generator().manual_seed(seed)
    q = {k: (dict(v) if isinstance(v, dict) else v) for k, v in p.items()}
    q["neuron_pool"] = dict(p["neuron_pool"], know_scale=torch.zeros(1))
    q["router"] = dict(p["router"], tau_attn={"kernel": 0.3 * torch.randn(cfg.d_model, 3, generator=g),
                                              "bias": torch.tensor([-0.6, -0.1, 0.3])})
    q["router"]["proj_attn"] = {"kernel": p["router"]["proj_attn"]["kernel"],
                                "bias": 0.5 * torch.randn(3 * cfg.d_route, generator=g)}
    return q


def _one_layer(cfg):
    return type(cfg)(**{**cfg.__dict__, "n_layers": 1})


def _attention_by_single_calls(p, cfg, ids):
    """The attention block of v41:1018-1082 written from single-route calls:
    h = LN(x) W + b split in three column blocks (Q, K, V in that order,
    :1019), tau columns 0 / 1 / 2 (:1022, :1036, :1053), Q and K each from
    fused_gate_srw on their own block times qk_scale (:1044-1045), V times
    v_scale, torch's causal scaled_dot_product_attention, then expand_O."""
    from oracle import srw_ref
    B, S = ids.shape
    D, dr, H = cfg.d_model, cfg.d_route, cfg.n_heads
    pool, rt, bp = p["neuron_pool"], p["router"], p["block_0"]
    x = p["token_emb"]["embedding"][ids] + p["pos_emb"]["embedding"][:S][None]
    n = F.layer_norm(x, (D,), bp["norm1"]["scale"], bp["norm1"]["bias"], eps=1e-6)
    h = n @ rt["proj_attn"]["kernel"] + rt["proj_attn"]["bias"]
    t = n @ rt["tau_attn"]["kernel"] + rt["tau_attn"]["bias"]
    one = lambda k, emb, rd, wr: srw_ref.fused_gate_srw(  # noqa: E731
        n, h[..., k * dr:(k + 1) * dr], emb, t[..., k:k + 1], rd, wr, max_chunk_size=cfg.max_chunk_size)[0]
    Q = one(0, pool["qk_emb"], pool["qk_read"], pool["qk_write"]) * pool["qk_scale"]
    K = one(1, pool["qk_emb"], pool["qk_read"], pool["qk_write"]) * pool["qk_scale"]
    V = one(2, pool["v_emb"], pool["v_read"], pool["v_write"]) * pool["v_scale"]
    hd = lambda u: u.reshape(B, S, H, D // H).transpose(1, 2)  # noqa: E731
    a = F.scaled_dot_product_attention(hd(Q), hd(K), hd(V), is_causal=True)
    x = x + a.transpose(1, 2).reshape(B, S, D) @ bp["attn"]["expand_O"]["kernel"]
    x = F.layer_norm(x, (D,), p["norm"]["scale"], p["norm"]["bias"], eps=1e-6)
    return x @ p["token_emb"]["embedding"].T


def _attn_block_mismatch(tiny):
    cfg, p = tiny
    cfg1 = _one_layer(cfg)
    q = _attn_params(cfg1, p, 21)
    ids = _ids(2, 11, cfg.vocab_size, 22)
    want = _attention_by_single_calls(q, cfg1, ids)
    got = dawn_ref.forward(q, cfg1, ids)
    return float((got - want).abs().max() / want.abs().max())


def test_attention_block_matches_single_route_formulation(tiny):
    """dawn_ref.forward's paired QK call, router split, tau columns and
    qk_scale placement against the block written from single-route calls
    and library attention (paired == two singles to ~1e-6)."""
    assert _attn_block_mismatch(tiny) < 1e-4


def _sign_flip_diff(tiny):
    cfg, p = tiny
    q = _attn_params(cfg, p, 23)
    ids = _ids(2, 9, cfg.vocab_size, 24)
    neg = dict(q, neuron_pool=dict(q["neuron_pool"], qk_scale=-q["neuron_pool"]["qk_scale"]))
    d_fwd = (dawn_ref.forward(q, cfg, ids) - dawn_ref.forward(neg, cfg, ids)).abs().max()
    d_pre = (dawn_ref.prefill(q, cfg, ids)[0] - dawn_ref.prefill(neg, cfg, ids)[0]).abs().max()
    return float(max(d_fwd, d_pre))


def test_qk_scale_sign_flip_leaves_logits_unchanged(tiny):
    """Q and K both carry qk_scale (v41:1044-1045, :1794-1797), so the
    attention logits Q K^T -- and everything after them -- are unchanged
    when qk_scale changes sign (the SRW outputs are linear in the scale), in
    forward and in prefill; a scale on one of the two flips every logit."""
    assert _sign_flip_diff(tiny) <= 1e-6


MODEL_MUTATIONS = {
    # h_Q and h_K blocks of the router taken in the wrong order
    "router_blocks_swapped": ("_route_blocks", lambda h, dr: (h[..., dr:2 * dr], h[..., :dr], h[..., 2 * dr:])),
    # tau columns of Q and K swapped
    "tau_columns_swapped": ("_tau_columns", lambda t: (t[..., 1:2], t[..., 0:1], t[..., 2:3])),
    # qk_scale applied to Q only
    "qk_scale_on_q_only": ("_qk_scaled", lambda QK, s: (QK[:, :, 0, :] * s, QK[:, :, 1, :])),
}


@pytest.mark.parametrize("name", sorted(MODEL_MUTATIONS))
def test_planted_router_and_scale_mistakes_are_caught(tiny, monkeypatch, name):
    attr, fn = MODEL_MUTATIONS[name]
    monkeypatch.setattr(dawn_ref, attr, fn)
    mis = _attn_block_mismatch(tiny)
    print(f"  {name}: block mismatch {mis:.2e}", flush=True)
    assert mis >= 1e-3
    if name == "qk_scale_on_q_only":
        assert _sign_flip_diff(tiny) > 1e-4
