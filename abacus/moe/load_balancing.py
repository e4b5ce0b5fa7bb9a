"""abacus.moe.load_balancing: the Switch-Transformer auxiliary loss (see abacus_amd.load_balancing)."""

from abacus_amd.load_balancing import load_balancing_loss

__all__ = ["load_balancing_loss"]
