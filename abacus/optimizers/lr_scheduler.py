"""abacus.optimizers.lr_scheduler: the warmup-stable-decay schedule (see abacus_amd.optim)."""

from abacus_amd.optim import WSD

__all__ = ["WSD"]
