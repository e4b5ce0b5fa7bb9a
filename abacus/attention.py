"""abacus.attention: the MoE decoder's attention (see abacus_amd.transformer)."""

from abacus_amd.transformer import MultiHeadAttention

__all__ = ["MultiHeadAttention"]
