"""GPU: the drop-in factories as trainable autograd nodes.

``make_sharded_srw(...)`` / ``make_sharded_srw_paired(...)`` return functions
whose outputs carry gradients the way jax.value_and_grad sees the
reference's (scripts/train_jax.py:586-603, 726): a loss built from out,
score_lb and dead_penalty backpropagates to x, h, emb, tau_offset, read and
write through srw_backward.  Compared with the oracle's hand-written VJP
(oracle/srw_vjp.py) on the same seeded inputs, 2e-2 relative (Frobenius).
"""

from __future__ import annotations

import pytest
import torch

from oracle import srw_vjp
from tests.parity import rel_fro

pytestmark = pytest.mark.gpu

BF = torch.bfloat16
D_LB, D_PEN = 0.37, -0.81


def _leaves(pkg, dev, B, S, D, dr, N, routes, seed):
    shape = pkg.inputs.PoolShape(T=B * S, D=D, N=N, dr=dr, routes=routes)
    inp = pkg.inputs.make_pool_inputs(shape, seed=seed)
    g = torch.Generator().manual_seed(seed + 3)
    tau = -0.5 + 0.2 * torch.randn(B * S, routes, generator=g)
    # bf16-valued float32 leaves: the factory's casts are then exact
    cpu = dict(x=inp["x"].to(BF).float().reshape(B, S, D),
               h=inp["h"].to(BF).float().reshape(B, S, dr) if routes == 1
               else inp["h"].to(BF).float().reshape(B, S, 2, dr),
               emb=inp["emb"].to(BF).float(),
               tau_offset=tau.reshape(B, S, 1) if routes == 1 else tau.reshape(B, S, 2, 1),
               read=inp["read"].to(BF).float(), write=inp["write"].to(BF).float())
    gpu = {k: v.to(dev).requires_grad_(True) for k, v in cpu.items()}
    return cpu, gpu


def _loss(outs, d_out):
    return (outs[0] * d_out).sum() + D_LB * outs[3] + D_PEN * outs[18]


def test_single_route_gradients_match_oracle(pkg, dev):
    B, S, D, dr, N = 2, 80, 384, 128, 2600
    print(f"[gpu] autograd single B{B} S{S} N{N}", flush=True)
    cpu, gpu = _leaves(pkg, dev, B, S, D, dr, N, 1, seed=41)
    fused = pkg.make_sharded_srw(max_chunk_size=1300)
    outs = fused(*(gpu[k] for k in ("x", "h", "emb", "tau_offset", "read", "write")))
    assert len(outs) == 22
    d_out = torch.randn(B, S, D, generator=torch.Generator().manual_seed(9))
    _loss(outs, d_out.to(dev)).backward()
    torch.cuda.synchronize()
    T = B * S
    ref = srw_vjp.fused_gate_srw_vjp(cpu["x"].reshape(T, D), cpu["h"].reshape(T, dr), cpu["emb"],
                                     cpu["tau_offset"].reshape(T, 1), cpu["read"], cpu["write"],
                                     d_out.reshape(T, D), D_LB, D_PEN, max_chunk_size=1300)
    pairs = dict(x="dx", h="dh", emb="demb", tau_offset="dtau_offset", read="dread", write="dwrite")
    for k, rk in pairs.items():
        got = gpu[k].grad
        assert got is not None and got.shape == gpu[k].shape and got.dtype == torch.float32, k
        err = rel_fro(got.cpu().reshape(ref[rk].shape), ref[rk].float())
        print(f"  {k}: rel err {err:.3e}", flush=True)
        assert err <= 2e-2, (k, err)


def test_paired_gradients_match_oracle(pkg, dev):
    B, S, D, dr, N = 2, 48, 384, 128, 1580
    print(f"[gpu] autograd paired B{B} S{S} N{N}", flush=True)
    cpu, gpu = _leaves(pkg, dev, B, S, D, dr, N, 2, seed=42)
    fused = pkg.make_sharded_srw_paired(max_chunk_size=2048)
    outs = fused(*(gpu[k] for k in ("x", "h", "emb", "tau_offset", "read", "write")))
    assert outs[0].shape == (B, S, 2, D)
    d_out = torch.randn(B, S, 2, D, generator=torch.Generator().manual_seed(10))
    _loss(outs, d_out.to(dev)).backward()
    torch.cuda.synchronize()
    T = B * S
    ref = srw_vjp.fused_gate_srw_vjp(cpu["x"].reshape(T, D).repeat_interleave(2, dim=0),
                                     cpu["h"].reshape(2 * T, dr), cpu["emb"],
                                     cpu["tau_offset"].reshape(2 * T, 1), cpu["read"], cpu["write"],
                                     d_out.reshape(2 * T, D), D_LB, D_PEN, max_chunk_size=N)
    want = dict(x=ref["dx"].reshape(T, 2, D).sum(dim=1).reshape(B, S, D), h=ref["dh"].reshape(B, S, 2, dr),
                emb=ref["demb"], tau_offset=ref["dtau_offset"].reshape(B, S, 2, 1), read=ref["dread"],
                write=ref["dwrite"])
    for k, v in want.items():
        err = rel_fro(gpu[k].grad.cpu(), v.float())
        print(f"  {k}: rel err {err:.3e}", flush=True)
        assert err <= 2e-2, (k, err)


def test_gradient_flags_of_the_outputs(pkg, dev):
    """Outputs behind stop_gradient in the reference, and the counts, carry no
    gradient; a loss through a differentiable diagnostic the backward does not
    cover raises instead of returning a silently wrong gradient."""
    B, S, D, dr, N = 1, 64, 128, 64, 500
    print(f"[gpu] autograd flags N{N}", flush=True)
    _, gpu = _leaves(pkg, dev, B, S, D, dr, N, 1, seed=43)
    fused = pkg.make_sharded_srw()
    outs = fused(*(gpu[k] for k in ("x", "h", "emb", "tau_offset", "read", "write")))
    # score_skew (13) and score_kurt (17) sit behind stop_gradient (v41:466-474)
    for i in (1, 2, 6, 7, 8, 10, 11, 12, 13, 14, 15, 17, 19, 20, 21):
        assert not outs[i].requires_grad, i
    for i in (0, 3, 4, 5, 9, 16, 18):
        assert outs[i].requires_grad, i
    with pytest.raises(NotImplementedError, match="score_std"):
        (outs[0].sum() + outs[4]).backward()
    torch.cuda.synchronize()
