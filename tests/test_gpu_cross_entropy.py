"""abacus_cross_entropy_fwd / _bwd and next_token_loss on the GPU (kernels/liger.py:12-47).

Against fp64 cross-entropy of the same logits: the mean loss within rtol 1e-5 (fp32
log-sum-exp), the gradient's normwise error no larger than torch's own cross_entropy in the
logits' dtype (which rounds the log-softmax to that dtype) plus a margin, ignored rows
exactly zero; vector and element-wise row paths (V a multiple of 8 or not); the
incoming gradient read from the device; and the decoder loss through the module path.
"""

import pytest
import torch
import torch.nn.functional as F

from abacus_amd import _lib
from abacus_amd.train import _CrossEntropyFunction, next_token_loss

pytestmark = pytest.mark.gpu


def _case(N, V, dtype, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    logits = (torch.randn(N, V, device="cuda", generator=g) * 3).to(dtype)
    targets = torch.randint(0, V, (N,), device="cuda", generator=g)
    targets[::7] = -100  # ignored rows
    return logits, targets


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("N,V", [(1000, 32000), (300, 1003), (5, 8)], ids=["V32000", "V1003_ragged", "tiny"])
def test_cross_entropy_matches_fp64(dtype, N, V):
    logits, targets = _case(N, V, dtype, seed=N + V)
    count = int((targets != -100).sum())
    x = logits.clone().requires_grad_()
    loss = _CrossEntropyFunction.apply(x, targets, count, -100)
    upstream = torch.tensor(0.75, device="cuda")
    (grad,) = torch.autograd.grad(loss, x, upstream)
    ref_x = logits.double().requires_grad_()
    ref = F.cross_entropy(ref_x, targets, ignore_index=-100)
    (ref_grad,) = torch.autograd.grad(ref, ref_x, upstream.double())
    assert abs(float(loss.detach()) - float(ref)) <= 1e-5 * abs(float(ref))
    assert torch.all(grad[targets == -100] == 0)
    t_x = logits.clone().requires_grad_()
    t_loss = F.cross_entropy(t_x, targets, ignore_index=-100)
    (t_grad,) = torch.autograd.grad(t_loss, t_x, upstream.to(dtype))
    err = float((grad.double() - ref_grad).norm() / ref_grad.norm())
    err_torch = float((t_grad.double() - ref_grad).norm() / ref_grad.norm())
    bound = 1e-5 if dtype == torch.float32 else max(1.25 * err_torch, 4e-3)
    assert err <= bound, f"normwise gradient error {err:.3g} (torch {err_torch:.3g})"


def test_next_token_loss_uses_kernels_and_matches_slice_form():
    torch.manual_seed(5)
    B, L, V = 2, 64, 32000
    tokens = torch.randint(0, V, (B, L), device="cuda")
    tokens[0, 10] = -100
    tokens[1, -1] = -100
    logits = torch.randn(B, L, V, device="cuda").to(torch.bfloat16).requires_grad_()
    timer = _lib.KernelTimer()
    with timer:
        loss = next_token_loss(logits, tokens)
        (grad,) = torch.autograd.grad(loss, logits)
    calls = timer.totals_ms()
    assert "abacus_cross_entropy_fwd" in calls and "abacus_cross_entropy_bwd" in calls
    assert loss.dtype == torch.bfloat16
    ref_x = logits.detach().double().requires_grad_()
    ref = F.cross_entropy(ref_x[:, :-1].reshape(-1, V), tokens[:, 1:].reshape(-1), ignore_index=-100)
    (ref_grad,) = torch.autograd.grad(ref, ref_x)
    assert abs(float(loss) - float(ref)) <= 2 ** -8 * abs(float(ref))  # the bf16 rounding of the loss
    err = float((grad.double() - ref_grad).norm() / ref_grad.norm())
    assert err < 4e-3, err
    assert torch.count_nonzero(grad[:, -1]) == 0


@pytest.mark.parametrize("bad", [32000, -3], ids=["past_vocab", "negative"])
def test_cross_entropy_flags_out_of_range_targets(bad):
    """kernels/liger.py:12-47 on GPU logits: a target outside [0, V) other than ignore_index makes the
    loss NaN, with no host sync (torch's GPU kernel stops on a device assertion), instead of a mean over
    the other rows; next_token_loss raises IndexError for it."""
    from abacus_amd.train import cross_entropy, next_token_loss

    logits, targets = _case(64, 32000, torch.bfloat16, seed=9)
    targets[5] = bad
    assert torch.isnan(cross_entropy(logits, targets))
    targets[5] = -100  # the ignore index itself is fine
    assert torch.isfinite(cross_entropy(logits, targets))
    tokens = targets.reshape(2, 32).clone()
    tokens[1, 7] = bad
    with pytest.raises(IndexError, match=str(bad)):
        next_token_loss(logits.reshape(2, 32, 32000), tokens)
