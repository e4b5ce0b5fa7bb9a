"""One training step of the MoE decoder on one GPU (the single-process path of trainer.py:58-97).

Clamp padding ids, forward, next-token cross-entropy with ignore_index -100,
backward, one AdamW step.  The optimizer is torch's AdamW with the reference
AdamW's defaults (lr 1e-3, betas (0.9, 0.999), eps 1e-8, weight decay 1e-2,
decoupled; optimizers/adamw.py:6-15, 85-119), its moment buffers in the
parameters' dtype like the reference's; on the GPU the fused single-pass form.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

__all__ = ["make_optimizer", "train_step"]


def make_optimizer(model: torch.nn.Module, lr: float = 1e-3) -> torch.optim.Optimizer:
    """torch's single-pass (fused) AdamW on GPU parameters: one read and write of each tensor per step."""
    fused = all(p.is_cuda for p in model.parameters())
    return torch.optim.AdamW(model.parameters(), lr=lr, betas=(0.9, 0.999), eps=1e-8, weight_decay=1e-2,
                             fused=fused)


def train_step(model: torch.nn.Module, optimizer: torch.optim.Optimizer, tokens_BL: torch.Tensor) -> torch.Tensor:
    """Returns the step's (detached) loss."""
    model.train()
    inputs_BL = tokens_BL.clamp(min=0)  # -100 is padding; the embedding has no row for it
    logits = model(inputs_BL)  # (B, L, vocab)
    targets = tokens_BL[:, 1:]
    if int((targets != -100).sum().item()) < 1:
        raise ValueError("batch has no target tokens")
    loss = F.cross_entropy(
        logits[:, :-1].reshape(-1, logits.size(-1)), targets.reshape(-1), ignore_index=-100,
    )
    optimizer.zero_grad(set_to_none=True)
    loss.backward()
    optimizer.step()
    return loss.detach()
