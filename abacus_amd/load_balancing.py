"""Switch-Transformer auxiliary loss on ROCm devices (abacus/moe/load_balancing.py:8-41).

Same signature, argument checks, error messages and result as the reference
`load_balancing_loss(router_probs, expert_indices, coeff=1e-2)`; the reduction
runs in the HIP kernels `abacus_moe_load_balancing_fwd` / `_bwd` (one HBM pass
over the probabilities, deterministic).  Gradients flow to `router_probs` only,
as in the reference, where the expert counts come from integer indices.
"""

from __future__ import annotations

import torch

from . import _lib
from .moe import _check_device

__all__ = ["load_balancing_loss"]


class _LoadBalancingLoss(torch.autograd.Function):
    @staticmethod
    def forward(ctx, probs_TE: torch.Tensor, slots_TK: torch.Tensor, coeff_e: float):
        T, E = probs_TE.shape
        K = slots_TK.shape[1]
        dev, dt = probs_TE.device, _lib.dtype_code(probs_TE.dtype, probs_TE.device)
        ws = torch.empty(_lib.query("abacus_moe_load_balancing_ws_bytes", T, E, device=dev), dtype=torch.uint8,
                         device=dev)
        f_E = torch.empty(E, dtype=torch.float32, device=dev)
        loss32 = torch.empty((), dtype=torch.float32, device=dev)
        loss = torch.empty((), dtype=probs_TE.dtype, device=dev)
        bad = torch.empty((), dtype=torch.int32, device=dev)
        _lib.call(
            "abacus_moe_load_balancing_fwd", _lib.ptr(probs_TE), _lib.ptr(slots_TK), T, E, K, coeff_e, dt,
            _lib.ptr(ws), _lib.ptr(f_E), _lib.ptr(loss32), _lib.ptr(loss), _lib.ptr(bad), _lib.stream_of(dev),
        )
        # torch.nn.functional.one_hot validates its classes the same way (and
        # synchronises to do it): negative ids first, then ids >= E
        flags = int(bad)
        if flags & 1:
            raise RuntimeError("Class values must be non-negative.")
        if flags & 2:
            raise RuntimeError("Class values must be smaller than num_classes.")
        ctx.save_for_backward(f_E)
        ctx.coeff_e, ctx.shape, ctx.dtype = coeff_e, (T, E), probs_TE.dtype
        return loss

    @staticmethod
    def backward(ctx, grad_loss):
        (f_E,) = ctx.saved_tensors
        T, E = ctx.shape
        dev = f_E.device
        # the loss and the probabilities share a dtype, and so do their gradients
        grad_loss = grad_loss.to(dtype=ctx.dtype).contiguous()
        dt = _lib.dtype_code(ctx.dtype)
        grad = torch.empty(T, E, dtype=ctx.dtype, device=dev)
        _lib.call(
            "abacus_moe_load_balancing_bwd", _lib.ptr(grad_loss), _lib.ptr(f_E), T, E, ctx.coeff_e, dt, _lib.ptr(grad),
            _lib.stream_of(dev),
        )
        return grad, None, None


def load_balancing_loss(
    router_probs: torch.Tensor,
    expert_indices: torch.Tensor,
    coeff: float = 1e-2,
) -> torch.Tensor:
    """Switch Transformer auxiliary loss (load_balancing.py:8-41)."""
    if router_probs.ndim < 1:
        raise ValueError("router_probs must include an expert dimension")
    n_experts = router_probs.shape[-1]
    if n_experts < 1:
        raise ValueError(f"router_probs has no experts, got shape {tuple(router_probs.shape)}")
    batch = router_probs.shape[:-1]
    if expert_indices.shape[: len(batch)] != batch:
        raise ValueError(
            f"expert_indices shape {tuple(expert_indices.shape)} does not match "
            f"router_probs batch {tuple(batch)}"
        )
    extra = expert_indices.ndim - len(batch)
    if extra > 1:
        raise ValueError(
            f"expert_indices has {extra} expert-choice dimensions, expected 0 or 1"
        )
    tokens = router_probs.numel() // n_experts
    if tokens == 0:
        return router_probs.new_zeros(())
    _check_device(router_probs, "load_balancing_loss")
    if expert_indices.device != router_probs.device:
        raise RuntimeError(
            f"expert_indices on {expert_indices.device} but router_probs on {router_probs.device}"
        )
    probs_TE = router_probs.reshape(tokens, n_experts)
    if not probs_TE.is_contiguous():
        probs_TE = probs_TE.contiguous()
    slots_TK = expert_indices.reshape(tokens, -1).to(dtype=torch.long).contiguous()
    if slots_TK.shape[1] == 0:  # the reference's amax over an empty slot dimension
        raise RuntimeError("amax(): Expected reduction dim 1 to have non-zero size.")
    # coeff * n_experts is a Python float that torch rounds to fp32 when it
    # multiplies the fp32 sum (load_balancing.py:40)
    return _LoadBalancingLoss.apply(probs_TE, slots_TK, float(coeff * n_experts))
