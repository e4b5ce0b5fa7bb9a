"""abacus.distributed.utils: process-group set-up that the training examples import
(abacus/distributed/utils.py:9-46).

Same names, arguments and behaviour as the reference's helpers: rank() and
world_size() are the process group's (torch.distributed raises when none is
initialised, as in the reference).  This build runs the MoE layer on one GPU, so the
multi-process paths that use these (data, tensor, pipeline and expert parallelism)
are not part of it; a single process needs none of them.
"""

from __future__ import annotations

import os
import sys

import torch
import torch.distributed as dist


def dist_env_vars() -> bool:
    """True when launched by torchrun (RANK and WORLD_SIZE set)."""
    return "RANK" in os.environ and "WORLD_SIZE" in os.environ


def init_process_group(backend: str = "gloo", device: torch.device | None = None) -> None:
    """One thread per process; gloo over the loopback interface, otherwise the backend on `device`."""
    torch.set_num_threads(1)
    if backend == "gloo":
        os.environ["GLOO_SOCKET_IFNAME"] = "lo0" if sys.platform == "darwin" else "lo"
        dist.init_process_group(backend=backend)
        return
    dist.init_process_group(backend=backend, device_id=device)


def shutdown() -> None:
    if dist.is_initialized():
        dist.destroy_process_group()


def rank() -> int:
    return dist.get_rank()


def world_size() -> int:
    return dist.get_world_size()


def print_peak_memory() -> None:
    """Peak device memory of this process (the reference prints nothing for the CPU)."""
    if not torch.cuda.is_available():
        return
    who = f"rank {rank()}" if dist.is_initialized() else "process"
    peak = torch.cuda.max_memory_allocated()
    print(f"{who} max CUDA memory {peak / 1024**2:.1f} MB", flush=True)


__all__ = ["dist_env_vars", "init_process_group", "shutdown", "rank", "world_size", "print_peak_memory"]
