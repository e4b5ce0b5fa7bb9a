"""float64 and float16 modules on CPU tensors (the host library): the reference's modules run in
whatever float dtype they are cast to (router.py:40-70, moe.py:60-86 are plain torch ops), so
`MoE(...).double()` and `.half()` must work here too.

- fp16 storage conversions against torch's casts: every binary16 value widened, and fp32 products
  rounded to binary16 (subnormals, overflow to infinity, ties), through the combine entry point.
- fp64 layer: routing bit-exact against the oracle given the library's logits (indices, counts,
  offsets, permutation, bias step; weights within a few ulp, the sigmoid's exp differing by an ulp
  between libm and torch), outputs and every gradient against the oracle's autograd in fp64
  (rtol 1e-12), and torch.autograd.gradcheck of the layer with respect to x and all four parameters.
- fp16 layer: routing bit-exact, outputs and gradients within 2e-2 of fp64.
- the load-balancing loss (computed in fp32 for every dtype, as the reference casts to float) and
  the router alone in both dtypes; GPU tensors of these dtypes are refused with a TypeError."""

import numpy as np
import pytest
import torch

from abacus.moe.load_balancing import load_balancing_loss
from abacus.moe.moe import MoE
from abacus.moe.router import Router
from abacus_amd import _lib
from oracle import moe_oracle as oracle


def _rel(got, want):
    return float((got.double() - want.double()).norm() / max(want.double().norm().item(), 1e-300))


def test_half_widening_is_exact_for_every_value():
    """combine_fwd with one slot of weight 1 copies y: every binary16 bit pattern (NaNs compared
    as NaN) comes back as torch widens it; -0 comes back +0, as the sum starts from +0."""
    bits = torch.arange(0, 1 << 16, dtype=torch.int32).to(torch.int16)
    y = bits.view(torch.float16).reshape(-1, 8)
    T, D = y.shape
    w = torch.ones(T, 1, dtype=torch.float16)
    idx = torch.zeros(T, 1, dtype=torch.int32)
    pos = torch.arange(T, dtype=torch.int32).reshape(T, 1)
    out = torch.empty_like(y)
    _lib.call("abacus_moe_combine_fwd", _lib.ptr(y), _lib.ptr(w), _lib.ptr(idx), _lib.ptr(pos), T, D, 1, _lib.F16,
              _lib.ptr(out), _lib.HOST)
    nan, zero = torch.isnan(y), y == 0
    assert torch.equal(torch.isnan(out), nan)
    keep = ~nan & ~zero
    assert torch.equal(out[keep].view(torch.int16), y[keep].view(torch.int16))
    assert torch.equal(out[zero].view(torch.int16), torch.zeros(int(zero.sum()), dtype=torch.int16))


@pytest.mark.parametrize("scale", [0.37, 3.0, 1e-3, 600.0, 1.0 / 3.0])
def test_half_rounding_matches_torch(scale):
    """fp32 products y * w rounded to binary16 (round to nearest even, subnormals, overflow to
    infinity) equal torch's (y.float() * w.float()).half() for every finite binary16 y (a zero
    product comes back +0)."""
    bits = torch.arange(0, 1 << 16, dtype=torch.int32).to(torch.int16)
    y = bits.view(torch.float16)
    y = y[torch.isfinite(y)].reshape(-1, 2)
    T, D = y.shape
    w = torch.full((T, 1), scale, dtype=torch.float16)
    idx = torch.zeros(T, 1, dtype=torch.int32)
    pos = torch.arange(T, dtype=torch.int32).reshape(T, 1)
    out = torch.empty_like(y)
    _lib.call("abacus_moe_combine_fwd", _lib.ptr(y), _lib.ptr(w), _lib.ptr(idx), _lib.ptr(pos), T, D, 1, _lib.F16,
              _lib.ptr(out), _lib.HOST)
    want = (y.float() * w.float()).half()
    nz = want != 0  # a zero comes back +0 (the sum starts from +0)
    assert torch.equal(out[nz].view(torch.int16), want[nz].view(torch.int16))
    assert torch.equal(out[~nz].view(torch.int16), torch.zeros(int((~nz).sum()), dtype=torch.int16))


def _layer(T, D, E, K, M, dtype, seed):
    torch.manual_seed(seed)
    moe = MoE(D, E, K, hidden_dim=M, bias_update_speed=1e-3, route_scale=1.5)
    with torch.no_grad():
        for p in (moe.router.w_DE, moe.w_gate_EDM, moe.w_up_EDM, moe.w_down_EMD):
            p.normal_(0.0, 0.3)
        moe.router.expert_bias_E.normal_(0.0, 0.05)
    x = torch.randn(T, D)
    target = torch.randn(T, D)
    return moe.to(dtype), x.to(dtype), target.to(dtype)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float16], ids=["fp64", "fp16"])
@pytest.mark.parametrize("T,D,E,K,M", [(96, 24, 8, 2, 40), (40, 12, 70, 9, 16)], ids=["small", "wide_E"])
def test_layer_matches_oracle(dtype, T, D, E, K, M):
    moe, x, target = _layer(T, D, E, K, M, dtype, seed=T + E)
    moe.train()
    bias0 = moe.router.expert_bias_E.detach().clone()
    xr = x.clone().requires_grad_()
    out = moe(xr)
    assert out.dtype == dtype
    ((out.double() - target.double()) ** 2).mean().backward()
    r = moe.router.last_routing

    w_o, idx_o, _ = oracle.route(r.logits_TE, bias0, K, moe.router.route_scale)
    assert torch.equal(r.indices_TK, idx_o)
    if dtype == torch.float64:
        torch.testing.assert_close(r.weights_TK, w_o, rtol=1e-14, atol=0)
    else:
        assert torch.equal(r.weights_TK, w_o)
    counts, offsets, perm, pos = oracle.dispatch(idx_o, E)
    assert np.array_equal(r.counts_E.numpy(), counts) and np.array_equal(r.offsets_E1.numpy(), offsets)
    assert np.array_equal(r.perm_R.numpy(), perm) and np.array_equal(r.pos_TK.numpy(), pos)
    assert torch.equal(moe.router.expert_bias_E, oracle.bias_step(bias0, idx_o, E, moe.router.bias_update_speed))

    params = {n: p.detach().double().requires_grad_() for n, p in moe.named_parameters()}
    x64 = x.double().requires_grad_()
    ref, _ = oracle.moe_forward(x64, params["router.w_DE"], bias0.double(), params["w_gate_EDM"],
                                params["w_up_EDM"], params["w_down_EMD"], K, moe.router.route_scale,
                                indices_TK=idx_o)
    ((ref - target.double()) ** 2).mean().backward()
    tol = 1e-12 if dtype == torch.float64 else 2e-2
    assert _rel(out.detach(), ref.detach()) < tol
    assert _rel(xr.grad, x64.grad) < tol
    for n, p in moe.named_parameters():
        assert p.grad.dtype == dtype
        assert _rel(p.grad, params[n].grad) < tol, n


def test_layer_gradcheck_fp64():
    """torch.autograd.gradcheck of MoE.forward (eval mode, so the bias stays put) with respect to x
    and all four parameters, on inputs whose selection values keep every top-k boundary at least
    1e-3 apart, far beyond gradcheck's perturbations."""
    T, D, E, K, M = 6, 5, 4, 2, 3
    for seed in range(100):
        moe, x, _ = _layer(T, D, E, K, M, torch.float64, seed)
        sel = torch.sigmoid(x @ moe.router.w_DE) + moe.router.expert_bias_E
        top = sel.sort(dim=-1, descending=True).values
        if float((top[:, K - 1] - top[:, K]).min()) > 1e-3:
            break
    else:
        pytest.fail("no seed gave well-separated routing")
    moe.eval()
    names = ["router.w_DE", "w_gate_EDM", "w_up_EDM", "w_down_EMD"]
    base = dict(moe.named_parameters())

    def f(xi, *ps):
        return torch.func.functional_call(moe, {**base, **dict(zip(names, ps))}, (xi,))

    inputs = (x.clone().requires_grad_(),) + tuple(base[n].detach().clone().requires_grad_() for n in names)
    assert torch.autograd.gradcheck(f, inputs, eps=1e-6, atol=1e-7, rtol=1e-6)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float16], ids=["fp64", "fp16"])
def test_router_alone_backward(dtype):
    torch.manual_seed(11)
    T, D, E, K = 50, 16, 8, 3
    router = Router(D, E, K, route_scale=1.5).to(dtype)
    x = torch.randn(T, D, dtype=dtype, requires_grad=True)
    g = torch.randn(T, K, dtype=dtype)
    router.eval()
    w, idx = router(x)
    assert w.dtype == dtype
    (w.double() * g.double()).sum().backward()
    x_ref = x.detach().double().requires_grad_()
    wde = router.w_DE.detach().double().requires_grad_()
    picked = torch.sigmoid(x_ref @ wde).gather(-1, idx)
    ((picked / picked.sum(-1, keepdim=True) * 1.5) * g.double()).sum().backward()
    tol = 1e-12 if dtype == torch.float64 else 2e-2
    assert _rel(x.grad, x_ref.grad) < tol and _rel(router.w_DE.grad, wde.grad) < tol


@pytest.mark.parametrize("dtype", [torch.float64, torch.float16], ids=["fp64", "fp16"])
def test_load_balancing(dtype):
    torch.manual_seed(5)
    probs = torch.rand(3, 70, 12).to(dtype).requires_grad_()
    idx = torch.randint(0, 12, (3, 70, 4))
    loss = load_balancing_loss(probs, idx)
    assert loss.dtype == dtype
    loss.backward()
    p2 = probs.detach().clone().requires_grad_()
    want = oracle.load_balancing_loss(p2, idx)
    want.backward()
    # the reference computes this loss in fp32 for every dtype (load_balancing.py:30)
    tol = 1e-5 if dtype == torch.float64 else 2e-3
    assert abs(float(loss) - float(want)) <= tol * abs(float(want))
    assert _rel(probs.grad, p2.grad) < (1e-6 if dtype == torch.float64 else 2e-3)


@pytest.mark.parametrize("dtype", [torch.float64, torch.float16])
def test_gpu_tensors_of_host_only_dtypes_are_refused(dtype):
    with pytest.raises(TypeError, match="CPU tensors"):
        _lib.dtype_code(dtype, torch.device("cuda", 0))
    assert _lib.dtype_code(dtype, torch.device("cpu")) in (_lib.F64, _lib.F16)
    with pytest.raises(TypeError):
        _lib.dtype_code(torch.int32)
