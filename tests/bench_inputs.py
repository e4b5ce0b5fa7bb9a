"""The exact inputs bench.py times, for the GPU parity tests: abacus_amd.workloads.build (the host
recipe: seeded module init, N(0, 0.02^2) weights, N(0, 1) x and target, the Zipf selection bias),
moved to the GPU once per workload and shared by the tests of one process.

Each fetch restores the router's selection bias to the recipe's value (a train-mode forward steps
it) and clears the gradients, so every test sees the module as bench.py's first step does."""

from __future__ import annotations

import torch

from abacus_amd import workloads as W

_cache: dict[str, tuple] = {}


def bench_inputs(wl: W.Workload, device: torch.device):
    """(module, x_BLD, target_BLD) of the workload recipe on `device`."""
    if wl.name not in _cache:
        print(f"[bench-inputs] building {wl.name} on the host (the benchmark's recipe)", flush=True)
        moe, x, target = W.build(wl)
        moe = moe.to(device)
        x, target = x.to(device), target.to(device)
        _cache[wl.name] = (moe, x, target, moe.router.expert_bias_E.detach().clone())
        print(f"[bench-inputs] {wl.name} ready", flush=True)
    moe, x, target, bias0 = _cache[wl.name]
    with torch.no_grad():
        moe.router.expert_bias_E.copy_(bias0)
    moe.zero_grad(set_to_none=True)
    return moe, x, target
