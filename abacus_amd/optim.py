"""AdamW for the MoE decoder's training step (abacus/optimizers/adamw.py:4-119) on the GPU.

Same constructor, validation, state layout ({"step", "exp_avg", "exp_avg_sq"}
per parameter, keyed by id, moments in the parameter's dtype) and per-element
arithmetic as the reference's AdamW; ``step()`` updates every GPU parameter with a
gradient in one pass per tensor group (``abacus_adamw_step``: one HIP launch
per 48 tensors) instead of eight tensor ops per parameter.  CPU parameters take
the reference's eight torch ops.  ZeRO's owned
slices and gradient shards (``owned``, ``grad_shards``) belong to the
reference's multi-GPU data parallelism and are not taken here.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib

__all__ = ["AdamW", "WSD"]


class AdamW:
    def __init__(
        self,
        model: torch.nn.Module,
        lr: float = 1e-3,
        betas: tuple[float, float] = (0.9, 0.999),
        eps: float = 1e-8,
        weight_decay: float = 1e-2,
        owned: dict[int, tuple[int, int]] | None = None,
        grad_shards: dict[int, torch.Tensor] | None = None,
    ):
        if lr < 0:
            raise ValueError(f"Invalid learning rate: {lr}")
        if eps < 0:
            raise ValueError(f"Invalid epsilon: {eps}")
        if not 0.0 <= betas[0] < 1.0 or not 0.0 <= betas[1] < 1.0:
            raise ValueError(f"Invalid betas: {betas}")
        if weight_decay < 0:
            raise ValueError(f"Invalid weight decay: {weight_decay}")
        if owned is not None or grad_shards is not None:
            raise NotImplementedError("ZeRO-sharded optimizer state needs several data-parallel ranks; "
                                      "abacus_amd runs on one GPU")
        self.params = list(model.parameters())
        self.lr = lr
        self.beta1 = betas[0]
        self.beta2 = betas[1]
        self.eps = eps
        self.weight_decay = weight_decay
        self.state: dict[int, dict[str, torch.Tensor | int]] = {}

    def zero_grad(self) -> None:
        for param in self.params:
            param.grad = None

    @torch.no_grad()
    def step(self) -> None:
        groups: dict[tuple[torch.dtype, torch.device], list[tuple[torch.Tensor, ...]]] = {}
        for param in self.params:
            grad = param.grad
            if grad is None:
                continue
            if grad.is_sparse:
                raise RuntimeError("AdamW does not support sparse gradients")
            state = self.state.get(id(param))
            if state is None:
                state = {
                    "step": 0,
                    "exp_avg": torch.zeros_like(param),
                    "exp_avg_sq": torch.zeros_like(param),
                }
                self.state[id(param)] = state
            state["step"] += 1
            if not param.is_cuda:
                self._step_cpu(param, grad, state)
                continue
            if not grad.is_contiguous() or grad.dtype != param.dtype:
                grad = grad.contiguous().to(param.dtype)
            groups.setdefault((param.dtype, param.device), []).append(
                (param, grad, state["exp_avg"], state["exp_avg_sq"], state["step"]))
        for (dtype, device), items in groups.items():
            n = len(items)
            ptrs = [(ctypes.c_void_p * n)(*[_lib.ptr(it[k]) for it in items]) for k in range(4)]
            numels = (ctypes.c_int64 * n)(*[it[0].numel() for it in items])
            steps = (ctypes.c_int64 * n)(*[it[4] for it in items])
            _lib.call("abacus_adamw_step", *ptrs, numels, steps, n, self.lr, self.beta1, self.beta2, self.eps,
                      self.weight_decay, _lib.dtype_code(dtype), _lib.stream_of(device))


    def _step_cpu(self, weight: torch.Tensor, grad: torch.Tensor, state: dict) -> None:
        """One parameter's update as the reference's op sequence (optimizers/adamw.py:107-119)."""
        exp_avg, exp_avg_sq = state["exp_avg"], state["exp_avg_sq"]
        if self.weight_decay != 0:
            weight.mul_(1 - self.lr * self.weight_decay)
        exp_avg.lerp_(grad, 1 - self.beta1)
        exp_avg_sq.mul_(self.beta2).addcmul_(grad, grad, value=1 - self.beta2)
        step_size = self.lr / (1 - self.beta1 ** state["step"])
        denom = exp_avg_sq.sqrt().div_((1 - self.beta2 ** state["step"]) ** 0.5).add_(self.eps)
        weight.addcdiv_(exp_avg, denom, value=-step_size)


class WSD:
    """Warmup-stable-decay learning rate (optimizers/lr_scheduler.py): linear warmup over the
    first 2% of steps, constant, then linear decay to 0 over the last 10%."""

    def __init__(self, total_steps: int, lr: float = 5e-4):
        if total_steps < 1:
            raise ValueError(f"total_steps must be at least 1, got {total_steps}")
        if lr < 0:
            raise ValueError(f"Invalid learning rate: {lr}")
        self.total_steps = total_steps
        self.lr = lr
        self.warmup_steps = total_steps * 2 // 100
        self.decay_steps = total_steps * 10 // 100
        self._step = 0

    def learning_rate(self, step: int) -> float:
        if step < 1 or step > self.total_steps:
            raise ValueError(f"step must be in 1..{self.total_steps}, got {step}")
        if self.warmup_steps > 0 and step <= self.warmup_steps:
            return self.lr * step / self.warmup_steps
        if self.decay_steps > 0 and step > self.total_steps - self.decay_steps:
            done = (step - (self.total_steps - self.decay_steps)) / self.decay_steps
            return self.lr * (1 - done)
        return self.lr

    def step(self) -> float:
        self._step += 1
        return self.learning_rate(self._step)
