"""abacus.transformer_block: the MoE decoder block (TransformerBlockMoe) (see abacus_amd.transformer)."""

from abacus_amd.transformer import TransformerBlockMoe

__all__ = ["TransformerBlockMoe"]
