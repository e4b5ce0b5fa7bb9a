"""Synthetic MoE-layer workloads (shapes, seeds and initialisation) for tests and the benchmark.

Construction, per workload:
  1. torch.manual_seed(seed)
  2. MoE(D, E, K, hidden_dim=M) built on the CPU (consumes the RNG in the
     module's own init order)
  3. under no_grad, router.w_DE, w_gate_EDM, w_up_EDM, w_down_EMD overwritten
     in that order with N(0, 0.02^2)
  4. x = randn(B, L, D), then target = randn(B, L, D)
  5. cast to bf16 where the workload says so
The skewed workload adds a Zipf(1.2) rank-order selection bias to
router.expert_bias_E: ranks r = 1..E assigned to experts by randperm(E) with a
generator seeded 3, bias[e] = 0.1 * (ln p_r(e) - mean ln p), p_r ~ r^-1.2.
"""

from __future__ import annotations

import dataclasses
import math

import torch


@dataclasses.dataclass(frozen=True)
class Workload:
    name: str
    batch: int
    seq: int
    dim: int
    n_experts: int
    top_k: int
    hidden: int
    dtype: torch.dtype
    seed: int
    backward: bool = True
    zipf_bias: bool = False

    @property
    def tokens(self) -> int:
        return self.batch * self.seq

    @property
    def rows(self) -> int:
        return self.tokens * self.top_k

    def gemm_flops(self) -> float:
        """Grouped-GEMM flops: 6*R*D*M forward, 18*R*D*M forward + backward."""
        return (18.0 if self.backward else 6.0) * self.rows * self.dim * self.hidden

    def elem_bytes(self) -> int:
        return 2 if self.dtype == torch.bfloat16 else 4

    def dispatch_bytes(self) -> int:
        """Read each token once, write each routed row, plus the int32 row index."""
        s = self.elem_bytes()
        return s * self.dim * (self.tokens + self.rows) + 4 * self.rows

    def combine_bytes(self) -> int:
        """Read each routed row and write each token, plus weights and row indices."""
        s = self.elem_bytes()
        return s * self.dim * (self.rows + self.tokens) + (s + 4) * self.rows

    def with_tokens(self, batch: int, seq: int) -> "Workload":
        return dataclasses.replace(self, batch=batch, seq=seq, name=f"{self.name}@T{batch * seq}")


TINY_F32 = Workload("tiny_f32", 2, 128, 128, 8, 2, 256, torch.float32, 0)
MID_F32 = Workload("mid_f32", 4, 2048, 1024, 16, 2, 2816, torch.float32, 1)
MIXTRAL_BF16 = Workload("mixtral_bf16", 2, 2048, 4096, 8, 2, 14336, torch.bfloat16, 2)
SKEW_BF16_T64 = Workload("skewed_bf16_T64", 1, 64, 2048, 64, 6, 1408, torch.bfloat16, 3, backward=False, zipf_bias=True)
SKEW_BF16_T512 = Workload("skewed_bf16_T512", 1, 512, 2048, 64, 6, 1408, torch.bfloat16, 3, backward=False, zipf_bias=True)
SKEW_BF16_T16K = Workload("skewed_bf16_T16384", 8, 2048, 2048, 64, 6, 1408, torch.bfloat16, 3, zipf_bias=True)

# A fine-grained layer (the Qwen3-30B-A3B MoE shape: d_model 2048, 128 experts, top-8, expert hidden
# 768), 4 x 2048 tokens: about 512 rows per expert, short expert products; not one of the reference's
# benchmark configurations, a measured point for many small experts.
FINE_BF16 = Workload("finegrained_bf16", 4, 2048, 2048, 128, 8, 768, torch.bfloat16, 5)

ALL = {w.name: w for w in (TINY_F32, MID_F32, MIXTRAL_BF16, SKEW_BF16_T64, SKEW_BF16_T512, SKEW_BF16_T16K, FINE_BF16)}


def zipf_bias(n_experts: int, scale: float = 0.1, s: float = 1.2, seed: int = 3) -> torch.Tensor:
    """Per-expert selection bias from Zipf(s) rank order (fp32)."""
    gen = torch.Generator().manual_seed(seed)
    ranks = torch.randperm(n_experts, generator=gen) + 1  # expert e gets rank ranks[e]
    logp = torch.tensor([-s * math.log(r) for r in ranks.tolist()], dtype=torch.float64)
    logp = logp - torch.logsumexp(logp, 0)
    return (scale * (logp - logp.mean())).to(torch.float32)


def build(w: Workload, moe_cls=None, device: str | torch.device = "cpu"):
    """Build (module, x_BLD, target_BLD) for a workload on the CPU, then move to `device`."""
    if moe_cls is None:
        from abacus_amd.moe import MoE as moe_cls  # noqa: N813
    torch.manual_seed(w.seed)
    moe = moe_cls(w.dim, w.n_experts, w.top_k, hidden_dim=w.hidden)
    with torch.no_grad():
        moe.router.w_DE.normal_(0.0, 0.02)
        moe.w_gate_EDM.normal_(0.0, 0.02)
        moe.w_up_EDM.normal_(0.0, 0.02)
        moe.w_down_EMD.normal_(0.0, 0.02)
        if w.zipf_bias:
            moe.router.expert_bias_E.copy_(zipf_bias(w.n_experts))
    x = torch.randn(w.batch, w.seq, w.dim)
    target = torch.randn(w.batch, w.seq, w.dim)
    moe = moe.to(device=device, dtype=w.dtype)
    return moe, x.to(device=device, dtype=w.dtype), target.to(device=device, dtype=w.dtype)


def build_on_device(w: Workload, device: torch.device, moe_cls=None):
    """Same shapes and distributions, drawn directly on the GPU (fast path for the benchmark).

    The values differ from build(): only the distribution is the same.
    """
    if moe_cls is None:
        from abacus_amd.moe import MoE as moe_cls  # noqa: N813
    with torch.device("meta"):
        moe = moe_cls(w.dim, w.n_experts, w.top_k, hidden_dim=w.hidden)
    moe = moe.to_empty(device=device).to(dtype=w.dtype)
    gen = torch.Generator(device=device).manual_seed(w.seed)
    with torch.no_grad():
        for p in (moe.router.w_DE, moe.w_gate_EDM, moe.w_up_EDM, moe.w_down_EMD):
            p.normal_(0.0, 0.02, generator=gen)
        moe.router.expert_bias_E.zero_()
        if w.zipf_bias:
            moe.router.expert_bias_E.copy_(zipf_bias(w.n_experts).to(device=device, dtype=w.dtype))
    x = torch.randn(w.batch, w.seq, w.dim, device=device, generator=gen).to(w.dtype)
    target = torch.randn(w.batch, w.seq, w.dim, device=device, generator=gen).to(w.dtype)
    return moe, x, target
