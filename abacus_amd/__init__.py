"""abacus_amd: the MoE layer of satyaki-up/abacus, rebuilt for AMD Instinct MI355X (gfx950).

Python host code on PyTorch-ROCm; the compute is libabacus_moe.so (hand-written
HIP kernels) called through a C ABI (include/abacus_moe.h).
"""

from abacus_amd.moe import MoE, MoEExpertParallel, Router, Routing

__all__ = ["MoE", "MoEExpertParallel", "Router", "Routing"]
