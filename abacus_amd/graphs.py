"""HIP-graph replay of an inference forward pass.

A decode-sized batch spends a noticeable part of each forward launching kernels
(the router's two passes, the dispatch, two expert GEMMs and the combine, plus the
Python and ctypes calls around them).  GraphedForward captures one eval-mode
forward of a module for a fixed input shape and replays it: every kernel of the
forward runs again, on the captured buffers, from one graph launch.

The forward's C entry points record no memset, copy or host synchronisation into
the stream, which is what capture requires.  The replayed output tensor is the
same object every call (overwritten by the next replay); so are the captured
forward's routing tensors, kept as `routing` (the module's `last_routing` is
whatever its last Python-level forward left).
"""

from __future__ import annotations

import torch


class GraphedForward:
    """`g = GraphedForward(module, example_x)`, then `g(x)` for inputs of example_x's shape."""

    def __init__(self, module: torch.nn.Module, example_x: torch.Tensor, warmup: int = 2):
        if module.training:
            raise ValueError("GraphedForward captures the eval-mode forward: call module.eval() first "
                             "(a training forward steps the router bias and keeps tensors for backward)")
        if not example_x.is_cuda:
            raise ValueError("GraphedForward needs a GPU input")
        self.module = module
        self.x = example_x.detach().clone()
        dev = self.x.device
        # warm up on a side stream (default priority), as capture requires
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.no_grad(), torch.cuda.stream(side):
            for _ in range(warmup):
                module(self.x)
        torch.cuda.current_stream(dev).wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.no_grad(), torch.cuda.graph(self.graph):
            self.out = module(self.x)
        router = getattr(module, "router", None)
        self.routing = getattr(router, "last_routing", None)

    def __call__(self, x: torch.Tensor) -> torch.Tensor:
        if x.shape != self.x.shape or x.dtype != self.x.dtype or x.device != self.x.device:
            raise ValueError(f"GraphedForward was captured for {tuple(self.x.shape)} {self.x.dtype} on "
                             f"{self.x.device}, got {tuple(x.shape)} {x.dtype} on {x.device}")
        self.x.copy_(x)
        self.graph.replay()
        return self.out
