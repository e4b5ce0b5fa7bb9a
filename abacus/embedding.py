"""abacus.embedding: the MoE decoder's embedding (see abacus_amd.transformer)."""

from abacus_amd.transformer import Embedding

__all__ = ["Embedding"]
