"""abacus.rope: the MoE decoder's rotary position embedding (see abacus_amd.transformer)."""

from abacus_amd.transformer import Rotary, apply_rotary_pos_emb, rotate_half

__all__ = ["Rotary", "rotate_half", "apply_rotary_pos_emb"]
