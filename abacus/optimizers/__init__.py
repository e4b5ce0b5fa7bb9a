"""abacus.optimizers: the decoder's optimizer (see abacus_amd.optim)."""

from abacus_amd.optim import AdamW

__all__ = ["AdamW"]
