"""abacus.trainer: Trainer and get_device, single-process (see abacus_amd.train)."""

from abacus_amd.train import Trainer, get_device

__all__ = ["Trainer", "get_device"]
