"""abacus.moe.moe: MoE and MoEExpertParallel on the MI355X kernels (see abacus_amd.moe)."""

from abacus_amd.moe import MoE, MoEExpertParallel

__all__ = ["MoE", "MoEExpertParallel"]
