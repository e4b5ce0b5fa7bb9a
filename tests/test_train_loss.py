"""The decoder step's next-token loss (trainer.py:77-85) on the CPU: the padded-target form
train.py uses equals the reference's slice form, loss and gradient, with -100 padding."""

import pytest
import torch
import torch.nn.functional as F

from abacus_amd.train import next_token_loss


def _reference_loss(logits, tokens):
    targets = tokens[:, 1:]
    return F.cross_entropy(logits[:, :-1].reshape(-1, logits.size(-1)), targets.reshape(-1), ignore_index=-100)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64], ids=["fp32", "fp64"])
def test_padded_targets_equal_reference_slice(dtype):
    torch.manual_seed(3)
    B, L, V = 3, 9, 13
    tokens = torch.randint(0, V, (B, L))
    tokens[0, 4] = -100
    tokens[1, -1] = -100
    tokens[2, 0] = -100  # never a target
    logits = torch.randn(B, L, V, dtype=dtype, requires_grad=True)
    got = next_token_loss(logits, tokens)
    (g_got,) = torch.autograd.grad(got, logits)
    want = _reference_loss(logits, tokens)
    (g_want,) = torch.autograd.grad(want, logits)
    torch.testing.assert_close(got, want, rtol=1e-6 if dtype == torch.float32 else 1e-12, atol=0)
    torch.testing.assert_close(g_got, g_want, rtol=1e-6 if dtype == torch.float32 else 1e-12, atol=1e-9)
    assert torch.count_nonzero(g_got[:, -1]) == 0  # the last position has no target


def test_no_targets_raises():
    tokens = torch.full((2, 5), -100)
    tokens[:, 0] = 1  # only the first position, which is never a target
    with pytest.raises(ValueError, match="no target tokens"):
        next_token_loss(torch.zeros(2, 5, 4), tokens)


def test_out_of_range_target_raises():
    tokens = torch.tensor([[1, 2, 7, 3]])
    with pytest.raises(IndexError, match="out of bounds"):
        next_token_loss(torch.zeros(1, 4, 5), tokens)
