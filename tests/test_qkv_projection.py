"""_QKVProjection: the q/k/v projections with one joint backward (attention.py:129-131).

fp64 gradcheck on the CPU, and equality with three plain products and their autograd
gradients, including outputs that receive no gradient and inputs that need none."""

import torch

from abacus_amd.transformer import _QKVProjection


def _inputs(dtype=torch.float64, B=2, L=3, D=8, H=2, K=4):
    g = torch.Generator().manual_seed(5)
    x = torch.randn(B, L, D, generator=g, dtype=dtype, requires_grad=True)
    ws = [torch.randn(D, H, K, generator=g, dtype=dtype, requires_grad=True) for _ in range(3)]
    return x, ws


def test_gradcheck_fp64():
    x, ws = _inputs()
    assert torch.autograd.gradcheck(lambda *a: _QKVProjection.apply(*a), (x, *ws))


def test_matches_three_products_and_missing_grads():
    x, ws = _inputs(torch.float32)
    B, L, D = x.shape
    _, H, K = ws[0].shape
    q, k, v = _QKVProjection.apply(x, *ws)
    plain = [(x @ w.reshape(D, H * K)).view(B, L, H, K) for w in ws]
    for a, b in zip((q, k, v), plain):
        torch.testing.assert_close(a, b, rtol=0, atol=0)
        assert a.is_contiguous()
    # only q and v feed the loss: k's slot of the joint gradient is zero
    dq, dv = torch.randn_like(q), torch.randn_like(v)
    got = torch.autograd.grad((q * dq).sum() + (v * dv).sum(), [x, *ws])
    want = torch.autograd.grad((plain[0] * dq).sum() + (plain[2] * dv).sum(), [x, *ws], allow_unused=True)
    torch.testing.assert_close(got[0], want[0], rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(got[1], want[1], rtol=1e-5, atol=1e-5)
    assert not got[2].any() and want[2] is None
    torch.testing.assert_close(got[3], want[3], rtol=1e-5, atol=1e-5)
    # weights frozen: only dx
    x2 = x.detach().requires_grad_()
    q, k, v = _QKVProjection.apply(x2, *(w.detach() for w in ws))
    (q.sum() + k.sum() + v.sum()).backward()
    want_dx = sum(w.detach().reshape(D, H * K).sum(1) for w in ws).expand(B, L, D)
    torch.testing.assert_close(x2.grad, want_dx, rtol=1e-5, atol=1e-5)
