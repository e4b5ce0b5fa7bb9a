"""abacus.transformer_moe: the MoE decoder (TransformerMoe) (see abacus_amd.transformer)."""

from abacus_amd.transformer import TransformerMoe

__all__ = ["TransformerMoe"]
