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

from .optim import AdamW

__all__ = ["make_optimizer", "next_token_loss", "train_step"]


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
    if int((targets != -100).sum().item()) < 1:
        raise ValueError("batch has no target tokens")
    targets_BL = F.pad(targets, (0, 1), value=-100)
    return F.cross_entropy(logits_BLV.reshape(-1, logits_BLV.size(-1)), targets_BL.reshape(-1), ignore_index=-100)


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
