"""Oracle: CPU restatement of abacus's AdamW step. TEST INFRASTRUCTURE ONLY.

Only tests/ may use this module, and only to check results -- never as part of
the product path.

It restates abacus/optimizers/adamw.py:85-119 (AdamW.step) element by element
in numpy fp32: the reference runs one tensor op per stage on the parameter's
dtype, so every intermediate is rounded to that dtype (round to nearest even
for bf16).  The fp32 forms are those of torch's device kernels, the ones the
reference runs on a GPU (measured on MI355X against torch's own lerp_,
addcmul_, addcdiv_ and div_): lerp fma(w, b-a, a) for |w| < 0.5 (else
b - (b-a)*(1-w)), addcmul fma(s, b*c, a), addcdiv fma(s, b/c, a), division by
a Python scalar as a product with its reciprocal (taken in double, then
rounded to fp32); every other op on its own.  torch's CPU kernels associate addcmul and addcdiv differently (one bf16
ulp apart on a few elements in a million).  Scalars are the reference's
double-precision values rounded to fp32.  fma32 is the correctly rounded
fp32 fused multiply-add, from an exact fp64 product and an exact two-sum.

Pinning (tests/test_oracle_adamw.py):
  fma32          - against exact rational arithmetic (fractions.Fraction) on random and
                   halfway-rounding cases
  fp32 steps     - torch.optim.AdamW (single-tensor, same op sequence) over 5 steps, rtol 1e-5
  bf16 steps     - the reference's tensor-op sequence run by torch on the CPU in bf16, over
                   5 steps: elements within one bf16 ulp, nearly all identical (the GPU test
                   compares the kernel with torch's device ops exactly)
  first step     - closed form: zero moments, wd = 0: each |update| is lr * |g| / (|g| + eps')
                   within the bf16 roundings
  weight decay   - g = 0 for a step from zero moments: p' = bf16(p * (1 - lr*wd)) exactly
"""

from __future__ import annotations

import math

import numpy as np

__all__ = ["bf16_round", "fma32", "adamw_step"]


def bf16_round(x: np.ndarray) -> np.ndarray:
    """fp32 -> nearest bf16 (ties to even; NaN kept NaN), returned as fp32."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32)
    return np.where(np.isnan(x), np.float32(np.nan), out).astype(np.float32)


def fma32(a, b, c) -> np.ndarray:
    """a*b + c rounded once to fp32 (nearest even), for fp32 inputs.

    The fp64 product of two fp32 values is exact; s = fl64(p + c) with err the
    exact remainder (two-sum).  Rounding s to fp32 is the correct rounding of
    p + c unless s lies exactly halfway between two fp32 values and err != 0:
    then the exact sum lies on err's side of that midpoint.
    """
    f64 = np.float64
    a, b, c = (np.asarray(x, dtype=np.float32).astype(f64) for x in (a, b, c))
    p = a * b
    s = p + c
    bb = s - p
    err = (p - (s - bb)) + (c - bb)
    r = s.astype(np.float32)
    r64 = r.astype(f64)
    toward = np.where(s > r64, np.nextafter(r, np.float32(np.inf)), np.nextafter(r, np.float32(-np.inf)))
    mid = (s != r64) & ((r64 + toward.astype(f64)) * 0.5 == s)
    out = np.where(mid & (err > 0), np.maximum(r, toward), r)
    out = np.where(mid & (err < 0), np.minimum(r, toward), out)
    return out.astype(np.float32)


def adamw_step(p, g, m, v, step: int, lr: float, beta1: float, beta2: float, eps: float, weight_decay: float,
               dtype: str):
    """One AdamW step for one tensor; p, g, m, v fp32 arrays holding values of `dtype`
    ("bf16" or "fp32"); step is the count after this step's increment.  Returns (p, m, v)."""
    f = np.float32
    r = bf16_round if dtype == "bf16" else (lambda x: np.asarray(x, dtype=np.float32))
    p, g, m, v = (np.asarray(t, dtype=np.float32) for t in (p, g, m, v))
    if weight_decay != 0:
        p = r(p * f(1.0 - lr * weight_decay))
    w = f(1.0 - beta1)
    if abs(w) < 0.5:
        m = r(fma32(w, g - m, m))
    else:
        m = r(g - (g - m) * (f(1.0) - w))
    v = r(v * f(beta2))
    v = r(fma32(f(1.0 - beta2), g * g, v))
    bc1 = 1.0 - math.pow(beta1, step)
    bc2 = 1.0 - math.pow(beta2, step)
    d = r(np.sqrt(v))
    d = r(d * f(1.0 / math.pow(bc2, 0.5)))
    d = r(d + f(eps))
    p = r(fma32(f(-(lr / bc1)), m / d, p))
    return p, m, v
