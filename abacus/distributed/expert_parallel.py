"""Process-group helpers the MoE callers import (abacus/distributed/expert_parallel.py:10-13,91-102).

Only the single-process pieces exist here: the all-to-all dispatch of expert
parallelism is not part of this single-GPU build.
"""

import torch
import torch.distributed as dist

from abacus_amd.moe import _rank_and_world_size


class _SumReplicatedGrads(torch.autograd.Function):
    """Identity forward; backward sums the gradient over ranks (a no-op with one process)."""

    @staticmethod
    def forward(ctx, tensor: torch.Tensor) -> torch.Tensor:
        return tensor

    @staticmethod
    def backward(ctx, grad: torch.Tensor) -> torch.Tensor:
        if _rank_and_world_size()[1] == 1:
            return grad
        out = grad.detach().clone()
        dist.all_reduce(out, op=dist.ReduceOp.SUM)
        return out


__all__ = ["_rank_and_world_size", "_SumReplicatedGrads"]
