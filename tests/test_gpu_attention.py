"""abacus_attention_fwd / _bwd: flash-style causal attention (attention.py:136-141) on the GPU.

Against an fp64 evaluation of the reference's materialised formula on the same bf16
inputs: the output's normwise error must be no larger than torch's own fused kernel's
(which also keeps scores in fp32) plus a margin, every row finite, and the saved
log-sum-exp must match fp64 logsumexp of the scaled scores.  The gradients of q, k and v
are held to fp64 autograd of the same formula the same way, against torch's fused
backward's error.
"""

import math

import pytest
import torch

from abacus_amd import _lib

pytestmark = pytest.mark.gpu


def _reference_fp64(q, k, v, scale):
    """(B, L, H, K) inputs -> (B, L, H, K) output and (B, H, L) natural logsumexp, in fp64."""
    qh, kh, vh = (t.double().permute(0, 2, 1, 3) for t in (q, k, v))
    s = (qh @ kh.transpose(-1, -2)) * scale
    L = s.shape[-1]
    s = s.masked_fill(torch.ones(L, L, dtype=torch.bool, device=s.device).triu(1), float("-inf"))
    lse = torch.logsumexp(s, dim=-1)
    out = torch.softmax(s, dim=-1) @ vh
    return out.permute(0, 2, 1, 3), lse


def _run(q, k, v, scale):
    B, L, H, K = q.shape
    o = torch.empty_like(q)
    lse = torch.empty(B, H, L, dtype=torch.float32, device=q.device)
    _lib.call("abacus_attention_fwd", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), B, L, H, K, scale, 1, _lib.ptr(o),
              _lib.ptr(lse), _lib.stream_of(q.device))
    return o, lse


SHAPES = [(1, 128, 1, 64), (2, 384, 3, 64), (3, 1152, 2, 64), (4, 2048, 16, 64)]
SHAPE_IDS = ["L128", "L384_H3", "L1152_odd_pairs", "decoder"]  # L1152: 9 query blocks, 4 pairs + 1


@pytest.mark.parametrize("shape", SHAPES, ids=SHAPE_IDS)
def test_attention_fwd_matches_fp64(shape):
    B, L, H, K = shape
    g = torch.Generator(device="cuda").manual_seed(7)
    q, k, v = (torch.randn(B, L, H, K, device="cuda", generator=g).to(torch.bfloat16) for _ in range(3))
    scale = 1.0 / math.sqrt(K)
    o, lse2 = _run(q, k, v, scale)
    torch.cuda.synchronize()
    want, want_lse = _reference_fp64(q, k, v, scale)
    assert torch.isfinite(o.float()).all()
    err = float((o.double() - want).norm() / want.norm())
    from torch.nn.attention import SDPBackend, sdpa_kernel
    with sdpa_kernel([SDPBackend.EFFICIENT_ATTENTION, SDPBackend.FLASH_ATTENTION]):
        t = torch.nn.functional.scaled_dot_product_attention(
            *(x.permute(0, 2, 1, 3) for x in (q, k, v)), is_causal=True).permute(0, 2, 1, 3)
    err_torch = float((t.double() - want).norm() / want.norm())
    assert err <= max(1.25 * err_torch, 4e-3), f"normwise error {err:.3g} (torch fused {err_torch:.3g})"
    lse = lse2.double() * math.log(2.0)
    assert float((lse - want_lse).abs().max()) < 1e-3


def _run_bwd(q, k, v, o, lse2, dout, scale):
    B, L, H, K = q.shape
    dq, dk, dv = (torch.empty_like(q) for _ in range(3))
    nbytes = _lib.query("abacus_attention_bwd_ws_bytes", B, L, H)
    ws = torch.empty(nbytes // 4, dtype=torch.float32, device=q.device)
    _lib.call("abacus_attention_bwd", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(o), _lib.ptr(dout),
              _lib.ptr(lse2), B, L, H, K, scale, 1, _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv), _lib.ptr(ws), nbytes,
              _lib.stream_of(q.device))
    return dq, dk, dv


@pytest.mark.parametrize("shape", SHAPES, ids=SHAPE_IDS)
def test_attention_bwd_matches_fp64(shape):
    B, L, H, K = shape
    g = torch.Generator(device="cuda").manual_seed(11)
    q, k, v, dout = (torch.randn(B, L, H, K, device="cuda", generator=g).to(torch.bfloat16) for _ in range(4))
    scale = 1.0 / math.sqrt(K)
    o, lse2 = _run(q, k, v, scale)
    dq, dk, dv = _run_bwd(q, k, v, o, lse2, dout, scale)
    torch.cuda.synchronize()
    leaves = [t.double().requires_grad_() for t in (q, k, v)]
    want, _ = _reference_fp64(*leaves, scale)
    want_grads = torch.autograd.grad(want, leaves, dout.double())
    from torch.nn.attention import SDPBackend, sdpa_kernel
    tl = [t.detach().clone().requires_grad_() for t in (q, k, v)]
    with sdpa_kernel([SDPBackend.EFFICIENT_ATTENTION, SDPBackend.FLASH_ATTENTION]):
        t = torch.nn.functional.scaled_dot_product_attention(
            *(x.permute(0, 2, 1, 3) for x in tl), is_causal=True).permute(0, 2, 1, 3)
    torch_grads = torch.autograd.grad(t, tl, dout)
    for name, got, ref, tg in zip("qkv", (dq, dk, dv), want_grads, torch_grads):
        assert torch.isfinite(got.float()).all(), name
        err = float((got.double() - ref).norm() / ref.norm())
        err_torch = float((tg.double() - ref).norm() / ref.norm())
        assert err <= max(1.25 * err_torch, 4e-3), f"d{name}: normwise error {err:.3g} (torch fused {err_torch:.3g})"


def test_attention_fwd_rejects_shapes():
    q = torch.zeros(1, 100, 1, 64, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError, match="multiple of 128"):
        _run(q, q, q, 0.125)
    q = torch.zeros(1, 128, 1, 32, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError, match="head_dim"):
        _run(q, q, q, 0.125)
    q = torch.zeros(1, 128, 1, 64, dtype=torch.bfloat16, device="cuda")
    lse = torch.zeros(1, 1, 128, device="cuda")
    with pytest.raises(RuntimeError, match="workspace"):
        _lib.call("abacus_attention_bwd", *([_lib.ptr(q)] * 5), _lib.ptr(lse), 1, 128, 1, 64, 0.125, 1,
                  *([_lib.ptr(q)] * 3), _lib.ptr(lse), 16, _lib.stream_of(q.device))


def test_attention_module_runs_flash_kernels_forward_and_backward(monkeypatch):
    """MultiHeadAttention runs abacus_attention_fwd and _bwd on the (B, L, H, K) layout, with
    and without autograd, and its output and every gradient agree with the same module on
    torch's fused attention to bf16 accuracy."""
    import copy

    from abacus_amd import transformer as tr
    torch.manual_seed(9)
    B, L, H, K = 2, 256, 4, 64
    attn = tr.MultiHeadAttention(H * K, H, K).to(torch.bfloat16).cuda()
    rot = copy.deepcopy(tr.Rotary(K)).to(torch.bfloat16).cuda()
    x = torch.randn(B, L, H * K, device="cuda").to(torch.bfloat16)
    dy = torch.randn(B, L, H * K, device="cuda").to(torch.bfloat16)

    def run():
        xi = x.clone().requires_grad_()
        attn.zero_grad(set_to_none=True)
        y = attn(xi, rot)
        y.backward(dy)
        return [y.detach().float(), xi.grad.float()] + [p.grad.float() for p in attn.parameters()]

    timer = _lib.KernelTimer()
    with timer:
        fast = run()
        with torch.no_grad():
            fast_ng = attn(x, rot)
    calls = timer.totals_ms()
    assert "abacus_attention_fwd" in calls and "abacus_attention_bwd" in calls, sorted(calls)
    monkeypatch.setattr(tr, "flash_attention_enabled", False)
    timer = _lib.KernelTimer()
    with timer:
        slow = run()
    assert "abacus_attention_fwd" not in timer.totals_ms()
    names = ["out", "dx"] + [n for n, _ in attn.named_parameters()]
    for name, a, b in zip(names, fast, slow):
        err = float((a - b).norm() / b.norm())
        assert err < 1e-2, f"{name}: {err:.3g}"
    assert torch.equal(fast_ng.float(), fast[0])
