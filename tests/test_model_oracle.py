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
