"""abacus.norm: the MoE decoder's norm (see abacus_amd.transformer)."""

from abacus_amd.transformer import RMSNorm

__all__ = ["RMSNorm"]
