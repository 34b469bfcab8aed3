"""Seeded synthetic inputs for the benchmark configurations.

Recipe (identical for tests, smoke and bench, generated on the CPU in
float32 with a seeded ``torch.Generator`` and only then cast and moved, so
the CPU checker and the GPU see bit-identical inputs):

* x ~ N(0, 1), RMS-normalised per row: x / sqrt(mean(x^2) + 1e-6);
* emb rows ~ N(0, 1/dr);
* read and write rows ~ N(0, 1/D), then L2-normalised;
* h = x when the score is x.E^T (d_route = d_model), otherwise
  h = x W_proj + b with W_proj ~ N(0, 1/D) (Flax lecun-normal Dense, the
  router of models/dawn_spatial_v41_exp.py:969-970) and b = 0;
* tau_offset = -0.5 per token (the v4.1 tau Dense: zero kernel, bias -0.5,
  :971-976), or a per-seed scalar calibrated so that a target fraction of
  units passes.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import torch

__all__ = ["PoolShape", "CONFIGS", "make_pool_inputs", "calibrate_tau_offset"]


@dataclass(frozen=True)
class PoolShape:
    """One SRW pool call: T tokens, d_model D, d_route dr, N units, R routes."""
    T: int
    D: int
    N: int
    dr: int
    routes: int = 1
    h_is_x: bool = False          # score = x . E^T (dr == D, one route)
    router: bool = False          # h = x W_proj + b
    pass_target: float | None = None   # calibrate tau_offset to this pass fraction
    note: str = ""


CONFIGS = {
    # the Know-pool layer (fp32 CPU-runnable; bf16 on the GPU)
    "know": PoolShape(T=4096, D=384, N=25200, dr=384, h_is_x=True,
                      note="configs[0]: Know pool, d=384, N=25200, T=4096 (8x512)"),
    # QK (paired) + V pools of one attention layer, bf16
    "qk": PoolShape(T=4096, D=384, N=1580, dr=384, routes=2,
                    note="configs[1]: shared QK pool, Q and K routed independently"),
    "v": PoolShape(T=4096, D=384, N=2600, dr=384, h_is_x=True,
                   note="configs[1]: V pool"),
    # decode-shaped, 64 single-token steps through the 40M pools
    "decode_know": PoolShape(T=64, D=384, N=25200, dr=128, router=True, pass_target=0.03,
                             note="configs[3]: decode Know pool, 3% pass"),
    "decode_qk": PoolShape(T=64, D=384, N=1580, dr=128, routes=2, router=True,
                           note="configs[3]: decode QK pool"),
    "decode_v": PoolShape(T=64, D=384, N=2600, dr=128, router=True,
                          note="configs[3]: decode V pool"),
    # scaled-up Know pool, 2% pass
    "scaled": PoolShape(T=16384, D=1024, N=100000, dr=1024, h_is_x=True, pass_target=0.02,
                        note="configs[4]: d=1024, N=100000, T=16384"),
}


def _rms_norm_rows(x: torch.Tensor) -> torch.Tensor:
    return x / torch.sqrt(torch.mean(x * x, dim=-1, keepdim=True) + 1e-6)


def _l2_norm_rows(x: torch.Tensor) -> torch.Tensor:
    return x / torch.linalg.vector_norm(x, dim=-1, keepdim=True)


def make_pool_inputs(shape: PoolShape, seed: int = 0, *, T: int | None = None,
                     N: int | None = None) -> dict:
    """CPU float32 inputs for one pool call.

    Returns dict(x [T,D], h [T,R,dr] (absent when h_is_x), emb [N,dr],
    tau_offset [T,R], read [N,D], write [N,D]).  ``T``/``N`` override the
    configured sizes (for parity tests at reduced size); the generator
    stream is laid out so that a smaller T is a prefix of the full one.
    """
    T = shape.T if T is None else T
    N = shape.N if N is None else N
    D, dr, R = shape.D, shape.dr, shape.routes
    g = torch.Generator().manual_seed(int(seed))
    # pools first (independent of T), then per-token tensors
    emb = torch.randn(N, dr, generator=g) / (dr ** 0.5)
    read = _l2_norm_rows(torch.randn(N, D, generator=g))
    write = _l2_norm_rows(torch.randn(N, D, generator=g))
    w_proj = torch.randn(D, R * dr, generator=g) / (D ** 0.5) if shape.router else None
    gt = torch.Generator().manual_seed(int(seed) * 1000003 + 17)
    x = _rms_norm_rows(torch.randn(T, D, generator=gt))
    out = dict(x=x, emb=emb, read=read, write=write)
    if shape.h_is_x:
        assert R == 1 and dr == D
    elif shape.router:
        out["h"] = (x @ w_proj).reshape(T, R, dr).contiguous()
    else:
        out["h"] = _rms_norm_rows(torch.randn(T, R, dr, generator=gt))
    out["tau_offset"] = torch.full((T, R), -0.5)
    return out


def calibrate_tau_offset(inp: dict, target: float, n_tokens: int = 256,
                         act_threshold: float = 0.5) -> float:
    """Scalar tau_offset so that ~``target`` of (token, unit) pairs pass.

    Uses the first ``n_tokens`` tokens, scores from bf16-rounded operands
    and per-token moments; bisection on the mean pass fraction of
    margin = s - (mean + t std) - act_threshold > 0.
    """
    x = inp["x"][:n_tokens]
    h = inp.get("h")
    bf = torch.bfloat16
    e = inp["emb"].to(bf).to(torch.float32)
    hs = (x if h is None else h[:n_tokens].reshape(-1, h.shape[-1])).to(bf).to(torch.float32)
    s = hs @ e.T
    mu = s.mean(dim=-1, keepdim=True)
    sd = s.std(dim=-1, keepdim=True, correction=0)
    lo, hi = -10.0, 10.0
    for _ in range(60):
        mid = 0.5 * (lo + hi)
        frac = ((s - (mu + mid * sd) - act_threshold) > 0).float().mean().item()
        if frac > target:
            lo = mid
        else:
            hi = mid
    return 0.5 * (lo + hi)
