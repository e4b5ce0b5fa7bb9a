"""abacus.optimizers.adamw: AdamW on the GPU (see abacus_amd.optim)."""

from abacus_amd.optim import AdamW

__all__ = ["AdamW"]
