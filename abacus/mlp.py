"""abacus.mlp.MLP: the dense SwiGLU block (abacus/mlp.py:18-38).

Not on the MoE hot path; it is the one-expert special case of the MoE layer
and the reference's own tests compare against it.
"""

import torch


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
        act_BLM = torch.nn.functional.silu(x_BLD @ self.w_gate_DM) * (x_BLD @ self.w_up_DM)
        return act_BLM @ self.w_down_MD  # (B, L, D)
