"""One training step of the MoE decoder on one GPU (the single-process path of trainer.py:58-97).

Clamp padding ids, forward, next-token cross-entropy with ignore_index -100,
backward, one AdamW step.  The optimizer is abacus_amd.optim.AdamW, the
reference AdamW (optimizers/adamw.py) with its defaults (lr 1e-3, betas
(0.9, 0.999), eps 1e-8, weight decay 1e-2, decoupled) and its per-op
rounding, as one HIP pass per group of tensors.

``Trainer`` and ``get_device`` mirror trainer.py's single-process API, and
``cross_entropy`` / ``set_use_liger`` mirror kernels/liger.py; on the GPU the
cross-entropy is this library's HIP kernel pair either way.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

import os

from . import _lib
from .optim import WSD, AdamW

__all__ = ["Trainer", "cross_entropy", "get_device", "make_optimizer", "next_token_loss", "set_use_liger",
           "train_step"]


class _CrossEntropyFunction(torch.autograd.Function):
    """sum over rows not ignored of lse(x_i) - x_i[t_i], divided by `count` (kernels/liger.py:12-47).

    The HIP forward reads each row of logits once (log-sum-exp in fp32) and
    saves lse; the backward writes g * (softmax - onehot) / count in one pass,
    g read on the device.  The reference's torch path rounds the log-softmax
    to the logits' dtype before the loss; here only the gradient is rounded,
    once.
    """

    @staticmethod
    def forward(ctx, logits_NV, targets_N, count, ignore_index: int):
        # count: the rows not ignored, a Python int or a device scalar tensor
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
        if torch.is_tensor(ctx.count):  # fold 1 / count into g on the device
            g, scale = (g.float() / ctx.count).contiguous(), 1.0
        else:
            g, scale = g.float().contiguous(), 1.0 / ctx.count
        d_logits = torch.empty_like(logits_NV)
        _lib.call("abacus_cross_entropy_bwd", _lib.ptr(logits_NV), _lib.ptr(targets_N), _lib.ptr(lse), _lib.ptr(g),
                  scale, N, V, ctx.ignore_index, _lib.dtype_code(logits_NV.dtype), _lib.ptr(d_logits),
                  _lib.stream_of(logits_NV.device))
        return d_logits, None, None, None


_use_liger = False


def set_use_liger(enabled: bool) -> None:
    """kernels/liger.py:7-9.  On the GPU both settings run the HIP kernels; with it set, CPU
    inputs raise, as the reference's liger path does."""
    global _use_liger
    _use_liger = enabled


def cross_entropy(input: torch.Tensor, target: torch.Tensor, weight: torch.Tensor | None = None,
                  size_average: bool | None = None, ignore_index: int = -100, reduce: bool | None = None,
                  reduction: str = "mean", label_smoothing: float = 0.0) -> torch.Tensor:
    """kernels/liger.py:12-47: torch.nn.functional.cross_entropy's signature and result.

    (N, V) GPU logits in fp32 or bf16 with the default options (mean over the rows whose
    target is not ignore_index, no class weights or label smoothing) take the HIP kernels.
    Everything else is torch's cross_entropy.  Nothing waits on the host: the row count stays
    on the device, and a target outside [0, V) other than ignore_index makes the loss NaN (torch's
    GPU kernel stops on a device assertion there; next_token_loss, which syncs once for its count,
    raises IndexError instead).
    """
    if _use_liger and input.device.type != "cuda":
        raise RuntimeError("Liger cross entropy needs a CUDA tensor")
    fused = (input.is_cuda and input.dim() == 2 and input.dtype in (torch.float32, torch.bfloat16)
             and target.dim() == 1 and target.shape[0] == input.shape[0] and weight is None
             and size_average is None and reduce is None and reduction == "mean" and label_smoothing == 0.0)
    if not fused:
        return F.cross_entropy(input, target, weight=weight, size_average=size_average, ignore_index=ignore_index,
                               reduce=reduce, reduction=reduction, label_smoothing=label_smoothing)
    t = target.to(torch.int64).contiguous()
    count = (t != ignore_index).sum().to(torch.float32)
    return _CrossEntropyFunction.apply(input.contiguous(), t, count, int(ignore_index)).to(input.dtype)


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


def get_device() -> torch.device:
    """trainer.py:21-26: the GPU of LOCAL_RANK (made current), or the CPU without one."""
    if not torch.cuda.is_available():
        return torch.device("cpu")
    local_rank = int(os.environ.get("LOCAL_RANK", "0"))
    torch.cuda.set_device(local_rank)
    return torch.device("cuda", local_rank)


class Trainer:
    """trainer.py:29-103, the single-process path: the model moved to the device, the
    reference's AdamW with its defaults, and the WSD schedule when total_steps is given.
    Data, pipeline and context parallelism need several processes and are refused."""

    def __init__(self, model: torch.nn.Module, parallel=None, pipeline=None, total_steps: int | None = None):
        if parallel is not None and pipeline is not None:
            raise ValueError("pipeline parallel does not use DataParallel")
        if parallel is not None or pipeline is not None:
            raise NotImplementedError("data and pipeline parallelism need several processes; abacus_amd runs on "
                                      "one GPU")
        self.device = get_device()
        self.model = model.to(self.device)
        self.parallel = None
        self.pipeline = None
        self.optimizer = AdamW(self.model)
        self.scheduler = WSD(total_steps) if total_steps is not None else None
        if self.scheduler is not None:
            self.optimizer.lr = self.scheduler.learning_rate(1)

    def step(self, tokens_BL: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """(loss, local loss), both the step's mean next-token cross-entropy on one process."""
        self.model.train()
        tokens_BL = tokens_BL.to(self.device)
        inputs_BL = tokens_BL.clamp(min=0)  # -100 is padding; the embedding has no row for it
        logits = self.model(inputs_BL)  # (B, L, vocab)
        loss = next_token_loss(logits, tokens_BL)
        self.optimizer.zero_grad()
        loss.backward()
        local_loss = loss.detach()
        self._optimizer_step()
        return loss.detach(), local_loss

    def _optimizer_step(self) -> None:
        if self.scheduler is not None:
            self.optimizer.lr = self.scheduler.step()
        self.optimizer.step()
