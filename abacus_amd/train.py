"""One training step of the MoE decoder on one GPU (the single-process path of trainer.py:58-97).

Clamp padding ids, forward, next-token cross-entropy with ignore_index -100,
backward, one AdamW step.  The optimizer is abacus_amd.optim.AdamW, the
reference AdamW (optimizers/adamw.py) with its defaults (lr 1e-3, betas
(0.9, 0.999), eps 1e-8, weight decay 1e-2, decoupled) and its per-op
rounding, as one HIP pass per group of tensors.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from . import _lib
from .optim import AdamW

__all__ = ["make_optimizer", "next_token_loss", "train_step"]


class _CrossEntropyFunction(torch.autograd.Function):
    """sum over rows not ignored of lse(x_i) - x_i[t_i], divided by `count` (kernels/liger.py:12-47).

    The HIP forward reads each row of logits once (log-sum-exp in fp32) and
    saves lse; the backward writes g * (softmax - onehot) / count in one pass,
    g read on the device.  The reference's torch path rounds the log-softmax
    to the logits' dtype before the loss; here only the gradient is rounded,
    once.
    """

    @staticmethod
    def forward(ctx, logits_NV, targets_N, count: int, ignore_index: int):
        N, V = logits_NV.shape
        dev = logits_NV.device
        lse = torch.empty(N, dtype=torch.float32, device=dev)
        loss_rows = torch.empty(N, dtype=torch.float32, device=dev)
        _lib.call("abacus_cross_entropy_fwd", _lib.ptr(logits_NV), _lib.ptr(targets_N), N, V, ignore_index,
                  _lib.dtype_code(logits_NV.dtype), _lib.ptr(lse), _lib.ptr(loss_rows), _lib.stream_of(dev))
        ctx.save_for_backward(logits_NV, targets_N, lse)
        ctx.count, ctx.ignore_index = count, ignore_index
        return loss_rows.sum() / count

    @staticmethod
    def backward(ctx, g):
        logits_NV, targets_N, lse = ctx.saved_tensors
        N, V = logits_NV.shape
        g = g.float().contiguous()
        d_logits = torch.empty_like(logits_NV)
        _lib.call("abacus_cross_entropy_bwd", _lib.ptr(logits_NV), _lib.ptr(targets_N), _lib.ptr(lse), _lib.ptr(g),
                  1.0 / ctx.count, N, V, ctx.ignore_index, _lib.dtype_code(logits_NV.dtype), _lib.ptr(d_logits),
                  _lib.stream_of(logits_NV.device))
        return d_logits, None, None, None


def make_optimizer(model: torch.nn.Module, lr: float = 1e-3) -> AdamW:
    """The reference's AdamW with its default hyperparameters (optimizers/adamw.py:6-15)."""
    return AdamW(model, lr=lr, betas=(0.9, 0.999), eps=1e-8, weight_decay=1e-2)


def next_token_loss(logits_BLV: torch.Tensor, tokens_BL: torch.Tensor) -> torch.Tensor:
    """Mean cross-entropy of logits[:, :-1] against tokens[:, 1:], ignoring -100 (trainer.py:77-85).

    Taken over every position with the last one's target set to the ignore
    index: the same (logit, target) pairs and count as the reference's slice,
    without copying the (B, L-1, vocab) slice forward and back.
    """
    targets = tokens_BL[:, 1:]
    V = logits_BLV.size(-1)
    valid = targets != -100
    bad = valid & ((targets < 0) | (targets >= V))
    count, n_bad = (int(v) for v in torch.stack([valid.sum(), bad.sum()]).tolist())  # one host sync
    if count < 1:
        raise ValueError("batch has no target tokens")
    if n_bad:
        raise IndexError(f"Target {int(targets[bad][0])} is out of bounds.")
    targets_BL = F.pad(targets, (0, 1), value=-100)
    logits_NV = logits_BLV.reshape(-1, V)
    if logits_NV.is_cuda and logits_NV.dtype in (torch.float32, torch.bfloat16):
        # HIP kernels; the loss in the logits' dtype, as torch's cross_entropy returns it
        loss = _CrossEntropyFunction.apply(logits_NV.contiguous(), targets_BL.reshape(-1).to(torch.int64).contiguous(),
                                           count, -100)
        return loss.to(logits_NV.dtype)
    return F.cross_entropy(logits_NV, targets_BL.reshape(-1), ignore_index=-100)


def train_step(model: torch.nn.Module, optimizer: AdamW, tokens_BL: torch.Tensor) -> torch.Tensor:
    """Returns the step's (detached) loss."""
    model.train()
    inputs_BL = tokens_BL.clamp(min=0)  # -100 is padding; the embedding has no row for it
    logits = model(inputs_BL)  # (B, L, vocab)
    loss = next_token_loss(logits, tokens_BL)
    optimizer.zero_grad()
    loss.backward()
    optimizer.step()
    return loss.detach()
