"""Parity helpers shared by the GPU tests: tolerances and the tie band.

Tolerances (from the hot path's contract):
  * float32 path vs the float32 restatement: relative Frobenius error of out
    <= 1e-5;
  * bf16 path vs the bf16 restatement: relative Frobenius error of out
    <= 2e-2 (and, per token row, <= 5e-2 of that row's norm);
  * passing set: identical outside a tie band |margin| <= delta, where
    delta covers one bf16 ulp of the score plus the tau difference (bf16),
    or 1e-5 * max(1, s_std) (float32); inside the band at most
    MIS_BASE + MIS_PER_PAIR * (rows x units) mismatches (plus, where the
    moments are computed another way on purpose -- Gram statistics -- every
    pair inside that known tau shift);
  * dense gate (every unit's fp32 gate): see gate_close.
"""

from __future__ import annotations

import torch

REL_F32 = 1e-5
REL_BF16 = 2e-2
ROW_REL_BF16 = 5e-2


def rel_fro(got: torch.Tensor, ref: torch.Tensor) -> float:
    got = got.double()
    ref = ref.double()
    return float((got - ref).norm() / ref.norm().clamp_min(1e-30))


def row_rel_max(got: torch.Tensor, ref: torch.Tensor) -> float:
    got = got.double().reshape(-1, got.shape[-1])
    ref = ref.double().reshape(-1, ref.shape[-1])
    num = (got - ref).norm(dim=-1)
    den = ref.norm(dim=-1).clamp_min(1e-30)
    return float((num / den).max())


def unpack_mask(words: torch.Tensor, N: int) -> torch.Tensor:
    """[..., W] int64 words -> [..., N] bool (bit n % 64 of word n // 64)."""
    w = words.cpu().to(torch.int64)
    bits = torch.arange(64, dtype=torch.int64)
    b = ((w.unsqueeze(-1) >> bits) & 1).bool()
    return b.reshape(*w.shape[:-1], -1)[..., :N]


def bf16_ulp(v: torch.Tensor) -> torch.Tensor:
    """One bf16 ulp at |v| (2^(e-7) for v in [2^e, 2^(e+1)))."""
    a = v.abs().clamp_min(2.0 ** -126)
    e = torch.floor(torch.log2(a))
    return torch.pow(2.0, e - 7)


# Mismatches allowed inside the tie band.  A pair flips only when its fp32
# score lies next to a bf16 rounding boundary (the matrix cores sum the 16-bit
# products in another order than the CPU) and its margin is within that ulp of
# zero, or when its margin is within the moments' fp32 summation difference
# of zero: measured 0 - 1 per test at up to 1.3e7 (row, unit) pairs.
MIS_BASE = 2
MIS_PER_PAIR = 2e-7


def check_pass_set(mask_got: torch.Tensor, margin_ref: torch.Tensor, delta: torch.Tensor):
    """Mismatches of the passing set must lie inside |margin_ref| <= delta.

    Returns (n_mismatch, n_outside_band)."""
    ref = margin_ref > 0
    mism = mask_got != ref
    outside = mism & (margin_ref.abs() > delta)
    return int(mism.sum()), int(outside.sum())


def assert_pass_set(mask_got: torch.Tensor, margin_ref: torch.Tensor, delta: torch.Tensor,
                    shift: torch.Tensor | None = None) -> int:
    """The passing-set bar: no mismatch outside the tie band ``delta`` (+
    ``shift``), and at most MIS_BASE + MIS_PER_PAIR per pair inside it, plus
    every pair with |margin| <= ``shift`` (a known tau shift, e.g. Gram
    moments of the unrounded scores).  Returns the mismatch count."""
    band = delta if shift is None else delta + shift
    n_mis, n_out = check_pass_set(mask_got, margin_ref, band)
    bound = MIS_BASE + MIS_PER_PAIR * margin_ref.numel()
    if shift is not None:
        bound += int((margin_ref.abs() <= shift).sum())
    print(f"  pass-set mismatches {n_mis} (outside tie band {n_out}; allowed in band {bound:.1f})",
          flush=True)
    assert n_out == 0, f"{n_out} passing-set mismatches outside the tie band ({n_mis} total)"
    assert n_mis <= bound, f"{n_mis} passing-set mismatches inside the tie band, more than {bound:.1f}"
    return n_mis


def gate_close(got: torch.Tensor, ref: torch.Tensor, h: torch.Tensor, emb: torch.Tensor) -> tuple[bool, int]:
    """Dense gates [T, N] of two correct evaluations: equal within rtol 1e-3,
    atol 1e-7 where the score is determined, else anything.

    The gate act x intensity with act = sigmoid(500 margin): an fp32
    evaluation of the exponent 500 log2(e) margin rounds by up to ~721 x 2^-24
    x (|s| + |tau| + thr) absolute, moving act by as much relative (rtol
    1e-3).  The score itself comes from a dot product summed in different
    orders: in bf16 (h, emb bf16) a score within the fp32 accumulation error
    bound 2 dr 2^-24 sum|h||e| of a bf16 rounding midpoint may round either
    way (one ulp, which the slope 500 amplifies without bound) and is left
    out; in fp32 that bound, times 721 ln 2, joins the relative tolerance.
    Returns (ok, number of gates compared)."""
    hh, ee = h.double(), emb.double()
    s64 = hh @ ee.T
    acc = 2 * hh.shape[-1] * 2.0 ** -24 * (hh.abs() @ ee.abs().T)
    if h.dtype == torch.bfloat16:
        sb = s64.to(torch.bfloat16).double()
        keep = (bf16_ulp(sb) / 2 - (s64 - sb).abs()) > 2 * acc
        rtol = torch.full_like(s64, 1e-3)
    else:
        keep = torch.ones_like(s64, dtype=torch.bool)
        rtol = 1e-3 + 721 * 0.7 * acc
    g, r = got.double(), ref.double()
    ok = bool((((g - r).abs() <= rtol * r.abs() + 1e-7) | ~keep).all())
    return ok, int(keep.sum())

