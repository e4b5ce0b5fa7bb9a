"""Pins the AdamW oracle (oracle/adamw_oracle.py) on the CPU: against torch.optim.AdamW in
fp32, against the reference's tensor-op sequence run by torch in bf16, and against closed
forms of the first step and of weight decay alone."""

import math
from fractions import Fraction

import numpy as np
import torch

from oracle.adamw_oracle import adamw_step, bf16_round, fma32

HP = dict(lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=1e-2)


def _reference_ops(p, g, m, v, step, lr, beta1, beta2, eps, weight_decay):
    """adamw.py:104-119 as torch tensor ops on p's dtype (in place on clones)."""
    p, m, v = p.clone(), m.clone(), v.clone()
    if weight_decay != 0:
        p.mul_(1 - lr * weight_decay)
    m.lerp_(g, 1 - beta1)
    v.mul_(beta2).addcmul_(g, g, value=1 - beta2)
    bc1 = 1 - beta1 ** step
    bc2 = 1 - beta2 ** step
    denom = v.sqrt().div_(bc2 ** 0.5).add_(eps)
    p.addcdiv_(m, denom, value=-(lr / bc1))
    return p, m, v


def test_bf16_round_ties_to_even_and_specials():
    x = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 1.0 + 2 ** -8 + 2 ** -20, -2.5, np.inf, -np.inf, 0.0],
                 dtype=np.float32)
    want = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    np.testing.assert_array_equal(bf16_round(x), want)
    assert np.isnan(bf16_round(np.array([np.nan], dtype=np.float32)))[0]
    r = np.random.default_rng(0).standard_normal(100000).astype(np.float32) * 1e3
    np.testing.assert_array_equal(bf16_round(r), torch.from_numpy(r).to(torch.bfloat16).float().numpy())


def _fma_exact(a, b, c):
    """Correctly rounded fp32 of a*b + c by exact rational arithmetic (ties to even)."""
    x = Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c))
    lo = np.float32(float(x))  # within one fp32 ulp of x; pick the nearest candidate exactly
    cands = [np.nextafter(lo, np.float32(-np.inf)), lo, np.nextafter(lo, np.float32(np.inf))]
    best = min(cands, key=lambda y: (abs(Fraction(float(y)) - x), int(np.float32(y).view(np.uint32)) & 1))
    return np.float32(best)


def test_fma32_is_correctly_rounded():
    rng = np.random.default_rng(4)
    a = rng.standard_normal(3000).astype(np.float32)
    b = rng.standard_normal(3000).astype(np.float32)
    c = (rng.standard_normal(3000) * 10.0 ** rng.integers(-6, 6, 3000)).astype(np.float32)
    # halfway cases: a*b + c lands exactly between two fp32 values, then nudged by a tiny product
    one = np.float32(1.0)
    half_ulp = np.float32(2.0 ** -24)
    a = np.concatenate([a, [one, one, one, half_ulp, half_ulp]]).astype(np.float32)
    b = np.concatenate([b, [half_ulp, half_ulp * 3, -half_ulp, one + np.float32(2.0 ** -23), one]]).astype(np.float32)
    c = np.concatenate([c, [one, one, one, one, one]]).astype(np.float32)
    got = fma32(a, b, c)
    want = np.array([_fma_exact(x, y, z) for x, y, z in zip(a, b, c)], dtype=np.float32)
    np.testing.assert_array_equal(got, want)


def test_fp32_steps_match_torch_adamw():
    torch.manual_seed(0)
    p0 = torch.randn(4096)
    grads = [torch.randn(4096) * (0.1 * (k + 1)) for k in range(5)]
    param = torch.nn.Parameter(p0.clone())
    opt = torch.optim.AdamW([param], lr=HP["lr"], betas=(HP["beta1"], HP["beta2"]), eps=HP["eps"],
                            weight_decay=HP["weight_decay"], foreach=False)
    p, m, v = p0.numpy().copy(), np.zeros(4096, np.float32), np.zeros(4096, np.float32)
    for k, g in enumerate(grads):
        param.grad = g.clone()
        opt.step()
        p, m, v = adamw_step(p, g.numpy(), m, v, k + 1, dtype="fp32", **HP)
        np.testing.assert_allclose(p, param.detach().numpy(), rtol=1e-5, atol=1e-7)
        st = opt.state[param]
        np.testing.assert_allclose(m, st["exp_avg"].numpy(), rtol=1e-6, atol=1e-9)
        np.testing.assert_allclose(v, st["exp_avg_sq"].numpy(), rtol=1e-6, atol=1e-12)


def test_bf16_steps_match_reference_op_sequence():
    """Every intermediate rounded to bf16, as the reference's separate ops do: within one
    bf16 ulp of torch's CPU run of the same ops (its CPU kernels associate some products
    differently from the device kernels the oracle follows), and nearly all identical."""
    torch.manual_seed(1)
    n = 1 << 15
    p_t = torch.randn(n).to(torch.bfloat16)
    m_t = torch.zeros(n, dtype=torch.bfloat16)
    v_t = torch.zeros(n, dtype=torch.bfloat16)
    p, m, v = (t.float().numpy() for t in (p_t, m_t, v_t))
    for step in range(1, 6):
        g_t = (torch.randn(n) * 10 ** (step - 3)).to(torch.bfloat16)
        p_t, m_t, v_t = _reference_ops(p_t, g_t, m_t, v_t, step, **HP)
        p, m, v = adamw_step(p, g_t.float().numpy(), m, v, step, dtype="bf16", **HP)
        for name, a, b in (("p", p, p_t), ("m", m, m_t), ("v", v, v_t)):
            b = b.float().numpy()
            ulp = np.abs(b) * 2.0 ** -7 + 1e-38
            assert np.all(np.abs(a - b) <= ulp), f"step {step} {name}: more than one bf16 ulp apart"
            assert np.mean(a == b) > 0.995, f"step {step} {name}: only {np.mean(a == b):.4f} identical"
        # keep both on the same state so each step is compared from equal inputs
        p_t, m_t, v_t = (torch.from_numpy(t).to(torch.bfloat16) for t in (p, m, v))


def test_first_step_closed_form():
    """Zero moments, no decay: m = bf16(0.1 g), v = bf16(0.001 g^2), and the update is
    -lr/0.1 * m / (sqrt(v)/sqrt(0.001) + eps) = -lr * sign(g) up to the bf16 roundings."""
    g = np.array([3.0, -0.5, 1e-3, -7.25, 0.0], dtype=np.float32)
    p0 = np.ones_like(g)
    hp = dict(HP, weight_decay=0.0)
    p, m, v = adamw_step(p0, g, np.zeros_like(g), np.zeros_like(g), 1, dtype="bf16", **hp)
    np.testing.assert_array_equal(m, bf16_round(np.float32(0.1) * g))
    np.testing.assert_array_equal(v, bf16_round(np.float32(0.001) * (g * g)))
    du = p - p0
    nz = g != 0
    # |m/d| is 1 within a few bf16 roundings; p = 1 - 1e-3 lands on the bf16 grid near 1 (ulp 2^-8)
    np.testing.assert_allclose(np.abs(du[nz]), np.abs(bf16_round(p0[nz] - hp["lr"]) - p0[nz]), atol=2 ** -8)
    assert du[~nz] == 0


def test_weight_decay_alone():
    """g = 0 from zero moments: m, v stay 0, d = eps, so p' = bf16(p * (1 - lr*wd)) exactly."""
    p0 = bf16_round(np.random.default_rng(2).standard_normal(1000).astype(np.float32) * 4)
    z = np.zeros_like(p0)
    p, m, v = adamw_step(p0, z, z, z, 3, dtype="bf16", **HP)
    np.testing.assert_array_equal(p, bf16_round(p0 * np.float32(1 - HP["lr"] * HP["weight_decay"])))
    assert not m.any() and not v.any()
    # fp32: the same identity without rounding
    p32, _, _ = adamw_step(p0, z, z, z, 3, dtype="fp32", **HP)
    np.testing.assert_array_equal(p32, p0 * np.float32(1 - HP["lr"] * HP["weight_decay"]))
    assert math.isclose(float(np.float32(1 - HP["lr"] * HP["weight_decay"])), 0.99999, rel_tol=1e-7)
