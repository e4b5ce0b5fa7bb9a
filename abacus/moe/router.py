"""abacus.moe.router: the fused sigmoid top-k Router (see abacus_amd.moe)."""

from abacus_amd.moe import Router

__all__ = ["Router"]
