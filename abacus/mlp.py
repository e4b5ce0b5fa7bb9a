"""abacus.mlp: the dense SwiGLU blocks (abacus/mlp.py:18-81).

Not on the MoE hot path.  MLP is the one-expert special case of the MoE layer
and the reference's own tests compare against it; MLPTensorParallel is here so
that the callers that import it (transformer_block.py:13) resolve.  With one
process it is MLP with the reference's tensor-parallel construction; its
multi-process paths (hidden units sharded over ranks, sequence parallelism) are
not part of this single-GPU build and raise NotImplementedError.
"""

import torch

from abacus_amd.moe import _rank_and_world_size


def _swiglu(x_BLD: torch.Tensor, w_gate_DM: torch.Tensor, w_up_DM: torch.Tensor,
            w_down_MD: torch.Tensor) -> torch.Tensor:
    act_BLM = torch.nn.functional.silu(x_BLD @ w_gate_DM) * (x_BLD @ w_up_DM)
    return act_BLM @ w_down_MD  # (B, L, D)


class MLP(torch.nn.Module):
    def __init__(self, dim: int, hidden_dim: int | None = None):
        super().__init__()
        self.dim = dim
        self.hidden_dim = dim if hidden_dim is None else hidden_dim
        self.w_gate_DM = torch.nn.Parameter(torch.empty(self.dim, self.hidden_dim))
        self.w_up_DM = torch.nn.Parameter(torch.empty(self.dim, self.hidden_dim))
        self.w_down_MD = torch.nn.Parameter(torch.empty(self.hidden_dim, self.dim))
        for w in (self.w_gate_DM, self.w_up_DM, self.w_down_MD):
            torch.nn.init.xavier_uniform_(w)

    def forward(self, x_BLD: torch.Tensor) -> torch.Tensor:
        return _swiglu(x_BLD, self.w_gate_DM, self.w_up_DM, self.w_down_MD)


class MLPTensorParallel(torch.nn.Module):
    """mlp.py:41-81 on one process: the full (D, M), (D, M), (M, D) weights drawn by xavier in
    the reference's order (so a seed gives MLP's values), kept whole (rank 0's slice of one rank)."""

    def __init__(self, dim: int, hidden_dim: int | None = None, sequence_parallel: bool = False):
        super().__init__()
        self.dim = dim
        self.hidden_dim = dim if hidden_dim is None else hidden_dim
        self.sequence_parallel = sequence_parallel
        self.rank, self.world_size = _rank_and_world_size()
        if self.world_size > 1:
            raise NotImplementedError(
                f"MLPTensorParallel over {self.world_size} processes: tensor parallelism is not part of "
                "abacus_amd, which runs on one GPU"
            )
        weights = [torch.empty(self.dim, self.hidden_dim), torch.empty(self.dim, self.hidden_dim),
                   torch.empty(self.hidden_dim, self.dim)]
        for w in weights:
            torch.nn.init.xavier_uniform_(w)
        self.w_gate_DM = torch.nn.Parameter(weights[0])
        self.w_up_DM = torch.nn.Parameter(weights[1])
        self.w_down_MD = torch.nn.Parameter(weights[2])

    def forward(self, x_BLD: torch.Tensor) -> torch.Tensor:
        return _swiglu(x_BLD, self.w_gate_DM, self.w_up_DM, self.w_down_MD)


__all__ = ["MLP", "MLPTensorParallel"]
