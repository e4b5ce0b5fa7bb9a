"""abacus.kernels.liger: cross_entropy and set_use_liger (see abacus_amd.train)."""

from abacus_amd.train import cross_entropy, set_use_liger

__all__ = ["cross_entropy", "set_use_liger"]
