"""MI355X MoE layer: abacus's ``Router``, ``MoE`` and ``MoEExpertParallel`` on HIP kernels.

Same constructors, parameter/buffer names and shapes, initialisation RNG order
and error messages as the reference modules (abacus/moe/router.py:12-70,
abacus/moe/moe.py:22-141); the forward and backward run entirely in
libabacus_moe.so (gfx950), called through ctypes on torch's current stream.

Shape suffixes follow the reference: B batch, L sequence, D model dim,
M expert hidden dim, E experts, K selected experts, T = B*L tokens,
R = T*K routed rows.
"""

from __future__ import annotations

import dataclasses

import torch
import torch.distributed as dist
import torch.nn.functional as F

from abacus_amd import _lib
from abacus_amd._lib import call, ptr, query


def _rank_and_world_size() -> tuple[int, int]:
    """(rank, world size) of the default process group, (0, 1) without one."""
    if dist.is_available() and dist.is_initialized():
        return dist.get_rank(), dist.get_world_size()
    return 0, 1


@dataclasses.dataclass
class Routing:
    """Routing decided by the last forward (kept for inspection and tests).

    logits_TE are the exact logits the top-k ran on (dtype of x); counts_E,
    offsets_E1, perm_R and pos_TK describe the expert-contiguous row order.
    """

    logits_TE: torch.Tensor
    weights_TK: torch.Tensor
    indices_TK: torch.Tensor
    counts_E: torch.Tensor | None = None
    offsets_E1: torch.Tensor | None = None
    perm_R: torch.Tensor | None = None
    pos_TK: torch.Tensor | None = None


def _check_device(x: torch.Tensor, what: str) -> None:
    """GPU tensors run on the HIP library, CPU tensors on its host build; nothing else is accepted."""
    if x.device.type not in ("cuda", "cpu"):
        raise RuntimeError(
            f"abacus_amd {what} runs on ROCm (HIP) GPUs and on the CPU; got a tensor on {x.device}."
        )


def _contig(t: torch.Tensor) -> torch.Tensor:
    t = t if t.is_contiguous() else t.contiguous()
    if t.data_ptr() % 16 != 0:
        t = t.clone()
    return t


def _router_fwd(x_TD, w_DE, bias_E, top_k, route_scale):
    """Launch the fused router; returns (logits, weights, indices, idx32, score, hist, wt), wt the
    transposed router weights the kernel made (the backward's un-permute reuses them)."""
    T, D = x_TD.shape
    E = w_DE.shape[1]
    dev, dt = x_TD.device, _lib.dtype_code(x_TD.dtype, x_TD.device)
    logits = torch.empty(T, E, dtype=x_TD.dtype, device=dev)
    weights = torch.empty(T, top_k, dtype=x_TD.dtype, device=dev)
    indices = torch.empty(T, top_k, dtype=torch.int64, device=dev)
    idx32 = torch.empty(T, top_k, dtype=torch.int32, device=dev)
    score = torch.empty(T, top_k, dtype=_lib.acc_dtype(x_TD.dtype), device=dev)
    hist = torch.empty(query("abacus_moe_hist_len", T, E, device=dev), dtype=torch.int32, device=dev)
    wt = torch.empty(query("abacus_moe_router_ws_bytes", D, E, dt, device=dev), dtype=torch.uint8, device=dev)
    call(
        "abacus_moe_router_fwd", ptr(x_TD), ptr(w_DE), ptr(bias_E), T, D, E, top_k, float(route_scale), dt,
        ptr(logits), ptr(weights), ptr(indices), ptr(idx32), ptr(score), ptr(hist), ptr(wt), _lib.stream_of(dev),
    )
    return logits, weights, indices, idx32, score, hist, wt


def _router_dgrad_wgrad(ctx_needs_x, ctx_needs_w, x_TD, w_DE, dlogit, idx32, pos, dxp, wt):
    """dx and dW_DE of the router GEMM (plus the un-permute of dxp when given); wt holds the
    forward's transposed router weights."""
    T, D = x_TD.shape
    E = w_DE.shape[1]
    K = idx32.shape[1]
    dev, dt = x_TD.device, _lib.dtype_code(x_TD.dtype, x_TD.device)
    s = _lib.stream_of(dev)
    dx = dw = None
    if ctx_needs_x:
        dx = torch.empty_like(x_TD)
        call(  # w_DE = NULL: wt already holds the transposed weights
            "abacus_moe_unpermute_bwd", ptr(dxp), ptr(dlogit), ptr(idx32), ptr(pos), None, ptr(wt),
            T, D, E, K, dt, ptr(dx), s,
        )
    if ctx_needs_w:
        dw = torch.empty_like(w_DE)
        nbytes = query("abacus_moe_router_wgrad_ws_bytes", T, D, E, dt, device=dev)
        partial = torch.empty(nbytes // 4, dtype=torch.float32, device=dev)
        call("abacus_moe_router_wgrad", ptr(x_TD), ptr(dlogit), ptr(idx32), T, D, E, K, dt, ptr(partial), ptr(dw), s)
    return dx, dw


class _RouterFunction(torch.autograd.Function):
    """Router.forward (router.py:40-51) as one fused kernel; backward through the gating."""

    @staticmethod
    def forward(ctx, x_TD, w_DE, bias_E, top_k, route_scale, record):
        logits, weights, indices, idx32, score, _, wt = _router_fwd(x_TD, w_DE, bias_E, top_k, route_scale)
        ctx.save_for_backward(x_TD, w_DE, weights, score, idx32, wt)
        ctx.route_scale = float(route_scale)
        ctx.mark_non_differentiable(indices)
        if record is not None:
            record["routing"] = Routing(logits, weights, indices)
        return weights, indices

    @staticmethod
    def backward(ctx, dweights, _dindices):
        x_TD, w_DE, weights, score, idx32, wt = ctx.saved_tensors
        T, K = weights.shape
        dev, dt = x_TD.device, _lib.dtype_code(x_TD.dtype, x_TD.device)
        dlogit = torch.empty(T, K, dtype=_lib.acc_dtype(x_TD.dtype), device=dev)
        dweights = _contig(dweights.to(weights.dtype))
        call(
            "abacus_router_gating_bwd", ptr(dweights), ptr(weights), ptr(score), T, K, ctx.route_scale, dt,
            ptr(dlogit), _lib.stream_of(dev),
        )
        dx, dw = _router_dgrad_wgrad(
            ctx.needs_input_grad[0], ctx.needs_input_grad[1], x_TD, w_DE, dlogit, idx32, None, None, wt
        )
        return dx, dw, None, None, None, None


class _MoEFunction(torch.autograd.Function):
    """MoE.forward (moe.py:60-86) fused: router -> dispatch -> grouped SwiGLU -> combine."""

    @staticmethod
    def forward(ctx, x_TD, w_DE, w_gate, w_up, w_down, bias_E, top_k, route_scale, bias_speed, need_grad, record):
        T, D = x_TD.shape
        E, _, M = w_gate.shape
        K = top_k
        R = T * K
        dev, dt = x_TD.device, _lib.dtype_code(x_TD.dtype, x_TD.device)
        s = _lib.stream_of(dev)
        logits, weights, indices, idx32, score, hist, wt = _router_fwd(x_TD, w_DE, bias_E, K, route_scale)
        base = torch.empty_like(hist)
        counts = torch.empty(E, dtype=torch.int32, device=dev)
        offsets = torch.empty(E + 1, dtype=torch.int32, device=dev)
        update = bias_speed is not None and bias_speed != 0
        pos = torch.empty(T, K, dtype=torch.int32, device=dev)
        perm = torch.empty(R, dtype=torch.int32, device=dev)
        xp = torch.empty(R, D, dtype=x_TD.dtype, device=dev)
        call(
            "abacus_moe_dispatch", ptr(hist), ptr(x_TD), ptr(idx32), T, D, E, K, ptr(bias_E) if update else None,
            float(bias_speed) if update else 0.0, dt, ptr(counts), ptr(offsets), ptr(pos), ptr(perm), ptr(xp),
            ptr(base), s,
        )
        gate = torch.empty(R, M, dtype=x_TD.dtype, device=dev) if need_grad else None
        up = torch.empty(R, M, dtype=x_TD.dtype, device=dev) if need_grad else None
        h = torch.empty(R, M, dtype=x_TD.dtype, device=dev)
        call(
            "abacus_moe_gateup_fwd", ptr(xp), ptr(w_gate), ptr(w_up), ptr(offsets), R, D, M, E, dt,
            ptr(gate), ptr(up), ptr(h), s,
        )
        y = torch.empty(R, D, dtype=x_TD.dtype, device=dev)
        ws_bytes = _lib.query("abacus_moe_down_fwd_ws_bytes", R, M, D, E, dt, device=dev)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes > 0 else None
        call("abacus_moe_down_fwd", ptr(h), ptr(w_down), ptr(offsets), R, M, D, E, dt, ptr(y), ptr(ws), ws_bytes, s)
        out = torch.empty(T, D, dtype=x_TD.dtype, device=dev)
        call("abacus_moe_combine_fwd", ptr(y), ptr(weights), ptr(idx32), ptr(pos), T, D, K, dt, ptr(out), s)
        if need_grad:
            ctx.save_for_backward(x_TD, w_DE, w_gate, w_up, w_down, xp, gate, up, h, y, weights, score, idx32, pos,
                                  offsets, wt)
        ctx.route_scale = float(route_scale)
        if record is not None:
            record["routing"] = Routing(logits, weights, indices, counts, offsets, perm, pos)
        return out

    @staticmethod
    def backward(ctx, dout):
        (x_TD, w_DE, w_gate, w_up, w_down, xp, gate, up, h, y, weights, score, idx32, pos,
         offsets, wt) = ctx.saved_tensors
        T, D = x_TD.shape
        E, _, M = w_gate.shape
        K = idx32.shape[1]
        R = T * K
        dev, dt = x_TD.device, _lib.dtype_code(x_TD.dtype, x_TD.device)
        s = _lib.stream_of(dev)
        needs = ctx.needs_input_grad
        dout = _contig(dout.to(x_TD.dtype))
        dy = torch.empty(R, D, dtype=x_TD.dtype, device=dev)
        dlogit = torch.empty(T, K, dtype=_lib.acc_dtype(x_TD.dtype), device=dev)
        call(
            "abacus_moe_combine_bwd", ptr(dout), ptr(y), ptr(weights), ptr(score), ptr(pos), T, D, K,
            ctx.route_scale, dt, ptr(dy), ptr(dlogit), s,
        )
        # Each data gradient and the weight gradient beside it go in one launch
        # when both are wanted (abacus_moe_down_bwd / abacus_moe_gateup_bwd).
        dgate = torch.empty(R, M, dtype=x_TD.dtype, device=dev)
        dup = torch.empty(R, M, dtype=x_TD.dtype, device=dev)
        dw_down = None
        if needs[4]:
            dw_down = torch.empty_like(w_down)
            call(
                "abacus_moe_down_bwd", ptr(dy), ptr(w_down), ptr(gate), ptr(up), ptr(h), ptr(offsets), R, M, D, E,
                dt, ptr(dgate), ptr(dup), ptr(dw_down), ptr(_lib.tile_ctr(dev)), s,
            )
        else:
            call(
                "abacus_moe_down_bwd_dgrad", ptr(dy), ptr(w_down), ptr(gate), ptr(up), ptr(offsets), R, M, D, E, dt,
                ptr(dgate), ptr(dup), s,
            )
        dxp = torch.empty(R, D, dtype=x_TD.dtype, device=dev) if needs[0] else None
        dw_gate = dw_up = None
        if needs[2] or needs[3]:
            dw_gate = torch.empty_like(w_gate)
            dw_up = torch.empty_like(w_up)
        if dxp is not None and dw_gate is not None:
            call(
                "abacus_moe_gateup_bwd", ptr(dgate), ptr(dup), ptr(w_gate), ptr(w_up), ptr(xp), ptr(offsets),
                R, D, M, E, dt, ptr(dxp), ptr(dw_gate), ptr(dw_up), ptr(_lib.tile_ctr(dev)), s,
            )
        elif dxp is not None:
            call(
                "abacus_moe_gateup_bwd_dgrad", ptr(dgate), ptr(dup), ptr(w_gate), ptr(w_up), ptr(offsets),
                R, D, M, E, dt, ptr(dxp), s,
            )
        elif dw_gate is not None:
            call(
                "abacus_moe_gateup_bwd_wgrad", ptr(xp), ptr(dgate), ptr(dup), ptr(offsets), R, D, M, E, dt,
                ptr(dw_gate), ptr(dw_up), ptr(_lib.tile_ctr(dev)), s,
            )
        dx, dw_DE = _router_dgrad_wgrad(needs[0], needs[1], x_TD, w_DE, dlogit, idx32, pos, dxp, wt)
        return (dx, dw_DE, dw_gate if needs[2] else None, dw_up if needs[3] else None, dw_down,
                None, None, None, None, None, None)


def _check_operands(x_BLD: torch.Tensor, *params: torch.Tensor) -> None:
    _check_device(x_BLD, "MoE")
    for p in params:
        if p.device != x_BLD.device:
            raise RuntimeError(f"MoE parameter on {p.device} but input on {x_BLD.device}")
        if p.dtype != x_BLD.dtype:
            raise RuntimeError(f"MoE parameter dtype {p.dtype} does not match input dtype {x_BLD.dtype}")
    _lib.dtype_code(x_BLD.dtype, x_BLD.device)


class Router(torch.nn.Module):
    """Sigmoid top-k router with DeepSeek-V3 auxiliary-loss-free balancing (router.py:12-70)."""

    def __init__(
        self,
        dim: int,
        n_experts: int,
        top_k: int,
        bias_update_speed: float = 1e-3,
        route_scale: float = 1.0,
        expert_parallel: bool = False,
    ):
        super().__init__()
        if n_experts < 1:
            raise ValueError(f"n_experts must be at least 1, got {n_experts}")
        if not 1 <= top_k <= n_experts:
            raise ValueError(f"top_k must be in [1, {n_experts}], got {top_k}")
        self.dim = dim
        self.n_experts = n_experts
        self.top_k = top_k
        self.bias_update_speed = bias_update_speed
        self.route_scale = route_scale
        self.expert_parallel = expert_parallel
        self.w_DE = torch.nn.Parameter(torch.empty(dim, n_experts))  # (D, E)
        torch.nn.init.xavier_uniform_(self.w_DE)
        self.register_buffer("expert_bias_E", torch.zeros(n_experts, dtype=self.w_DE.dtype))
        self.last_routing: Routing | None = None

    def forward(self, x_BLD: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        if self.expert_parallel and _rank_and_world_size()[1] > 1:
            raise NotImplementedError("expert parallelism across GPUs is not part of the single-GPU abacus_amd build")
        _check_operands(x_BLD, self.w_DE, self.expert_bias_E)
        lead = x_BLD.shape[:-1]
        x_TD = _contig(x_BLD.reshape(-1, self.dim))
        record: dict = {}
        if x_TD.shape[0] == 0:
            weights = x_BLD.new_empty(*lead, self.top_k)
            indices = torch.empty(*lead, self.top_k, dtype=torch.int64, device=x_BLD.device)
        else:
            weights, indices = _RouterFunction.apply(
                x_TD, self.w_DE, self.expert_bias_E, self.top_k, self.route_scale, record
            )
            self.last_routing = record["routing"]
            weights = weights.reshape(*lead, self.top_k)
            indices = indices.reshape(*lead, self.top_k)
        if self.training:
            self.update_bias(indices)
        return weights, indices

    @torch.no_grad()
    def update_bias(self, indices_BLK: torch.Tensor) -> None:
        """bias += speed * sign(sum(counts) - E * counts) in the bias dtype (router.py:57-70)."""
        if self.bias_update_speed == 0:
            return
        bias = self.expert_bias_E
        _check_device(bias, "Router.update_bias")
        idx = _contig(indices_BLK.reshape(-1).to(device=bias.device, dtype=torch.int64))
        call(
            "abacus_router_update_bias", ptr(idx), idx.numel(), self.n_experts, float(self.bias_update_speed),
            _lib.dtype_code(bias.dtype, bias.device), ptr(bias), _lib.stream_of(bias.device),
        )


def _init_expert_weights(n_experts: int, dim: int, hidden: int):
    """Per-expert interleaved xavier init: gate[e], up[e], down[e] for e = 0.. (moe.py:48-54)."""
    gate_EDM = torch.empty(n_experts, dim, hidden)
    up_EDM = torch.empty(n_experts, dim, hidden)
    down_EMD = torch.empty(n_experts, hidden, dim)
    for expert in range(n_experts):
        torch.nn.init.xavier_uniform_(gate_EDM[expert])
        torch.nn.init.xavier_uniform_(up_EDM[expert])
        torch.nn.init.xavier_uniform_(down_EMD[expert])
    return gate_EDM, up_EDM, down_EMD


def _run_router_pre_hooks(router: torch.nn.Module, x_BLD: torch.Tensor) -> None:
    """Forward pre-hooks registered on moe.router, called as the reference's self.router(x) would
    (moe.py:64).  The layer routes inside its fused kernels, so a hook may observe the input but not
    replace it."""
    for hid, hook in list(router._forward_pre_hooks.items()):
        if router._forward_pre_hooks_with_kwargs.get(hid, False):
            res = hook(router, (x_BLD,), {})
        else:
            res = hook(router, (x_BLD,))
        if res is not None:
            raise NotImplementedError("a forward pre-hook on moe.router may not replace the router's input: "
                                      "the MoE layer routes inside its fused kernels")


def _run_router_hooks(router: torch.nn.Module, x_BLD: torch.Tensor, weights_TK: torch.Tensor,
                      indices_TK: torch.Tensor, lead) -> None:
    """Forward hooks registered on moe.router, called with the router's output for this call,
    (weights_BLK, indices_BLK) (router.py:40-54), after the bias step as in the reference.  The weights
    are the routing the layer used, without a gradient path of their own (the layer's gradients flow
    through its fused node); a hook may observe them but not replace them."""
    k = indices_TK.shape[-1]
    output = (weights_TK.reshape(*lead, k), indices_TK.reshape(*lead, k))
    for hid, hook in list(router._forward_hooks.items()):
        if router._forward_hooks_with_kwargs.get(hid, False):
            res = hook(router, (x_BLD,), {}, output)
        else:
            res = hook(router, (x_BLD,), output)
        if res is not None:
            raise NotImplementedError("a forward hook on moe.router may not replace the router's output: "
                                      "the MoE layer routes inside its fused kernels")


class MoE(torch.nn.Module):
    """Top-k mixture of SwiGLU experts (moe.py:22-86) on MI355X kernels."""

    def __init__(
        self,
        dim: int,
        n_experts: int,
        top_k: int,
        hidden_dim: int | None = None,
        bias_update_speed: float = 1e-3,
        route_scale: float = 1.0,
    ):
        super().__init__()
        self.dim = dim
        self.n_experts = n_experts
        self.top_k = top_k
        self.hidden_dim = dim if hidden_dim is None else hidden_dim
        if self.hidden_dim < 1:
            raise ValueError(f"hidden_dim must be at least 1, got {self.hidden_dim}")
        self.router = Router(
            dim,
            n_experts,
            top_k,
            bias_update_speed=bias_update_speed,
            route_scale=route_scale,
        )
        gate_EDM, up_EDM, down_EMD = _init_expert_weights(n_experts, dim, self.hidden_dim)
        self.w_gate_EDM = torch.nn.Parameter(gate_EDM)  # (E, D, M)
        self.w_up_EDM = torch.nn.Parameter(up_EDM)  # (E, D, M)
        self.w_down_EMD = torch.nn.Parameter(down_EMD)  # (E, M, D)

    def forward(self, x_BLD: torch.Tensor) -> torch.Tensor:
        """Routes, dispatches, runs the experts and combines in one autograd node.

        Uses only attributes that MoEExpertParallel also defines, because its
        single-process forward calls this function unbound (moe.py:140-141).
        """
        router = self.router
        _check_operands(x_BLD, router.w_DE, router.expert_bias_E, self.w_gate_EDM, self.w_up_EDM, self.w_down_EMD)
        if router._forward_pre_hooks:
            _run_router_pre_hooks(router, x_BLD)
        batch_shape = x_BLD.shape[:-1]
        x_TD = x_BLD.reshape(-1, self.dim)
        if x_TD.shape[0] == 0:  # the reference routes the empty batch too (moe.py:64-70)
            if router._forward_hooks:
                empty_w = x_BLD.new_empty(0, self.top_k)
                empty_i = torch.empty(0, self.top_k, dtype=torch.int64, device=x_BLD.device)
                _run_router_hooks(router, x_BLD, empty_w, empty_i, batch_shape)
            return x_BLD
        x_TD = _contig(x_TD)
        record: dict = {}
        speed = router.bias_update_speed if router.training else None
        operands = (x_TD, router.w_DE, _contig(self.w_gate_EDM), _contig(self.w_up_EDM), _contig(self.w_down_EMD))
        D, M = self.dim, self.w_gate_EDM.shape[2]
        vec = 16 // x_TD.element_size()  # the GPU kernels move rows in 16-byte vectors
        Dp, Mp = -(-D // vec) * vec, -(-M // vec) * vec
        padded = x_TD.is_cuda and (Dp != D or Mp != M)
        if padded:
            # D and M zero-padded to whole vectors: zero columns of x and rows of w_DE add exact
            # zeros to the logits; a zero hidden unit has silu(0) * 0 = 0 and meets a zero row of
            # w_down; F.pad's backward slices the gradients back to the parameters' shapes.
            x_p, w_DE, w_gate, w_up, w_down = operands
            operands = (F.pad(x_p, (0, Dp - D)), F.pad(w_DE, (0, 0, 0, Dp - D)), F.pad(w_gate, (0, Mp - M, 0, Dp - D)),
                        F.pad(w_up, (0, Mp - M, 0, Dp - D)), F.pad(w_down, (0, Dp - D, 0, Mp - M)))
        need_grad = torch.is_grad_enabled() and any(t.requires_grad for t in operands)
        out_TD = _MoEFunction.apply(
            *operands, router.expert_bias_E, self.top_k, router.route_scale, speed, need_grad, record,
        )
        if padded:
            out_TD = out_TD[:, :D]
        router.last_routing = record["routing"]
        if router._forward_hooks:
            _run_router_hooks(router, x_BLD, record["routing"].weights_TK, record["routing"].indices_TK, batch_shape)
        return out_TD.reshape(*batch_shape, self.dim)  # (B, L, D)


class MoEExpertParallel(torch.nn.Module):
    """Top-k SwiGLU experts, one expert per rank (moe.py:89-161).

    With one process it holds every expert and runs MoE.forward; the
    multi-GPU all-to-all path is not part of this single-GPU build.
    """

    def __init__(
        self,
        dim: int,
        n_experts: int,
        top_k: int,
        hidden_dim: int | None = None,
        bias_update_speed: float = 1e-3,
        route_scale: float = 1.0,
    ):
        super().__init__()
        self.dim = dim
        self.n_experts = n_experts
        self.top_k = top_k
        self.hidden_dim = dim if hidden_dim is None else hidden_dim
        if self.hidden_dim < 1:
            raise ValueError(f"hidden_dim must be at least 1, got {self.hidden_dim}")
        self.rank, self.world_size = _rank_and_world_size()
        if self.world_size > 1 and self.n_experts != self.world_size:
            raise ValueError(
                f"expert parallel keeps 1 expert on each rank, "
                f"got {self.n_experts} experts and world size {self.world_size}"
            )
        if self.world_size > 1:
            raise NotImplementedError("expert parallelism across GPUs is not part of the single-GPU abacus_amd build")
        self.router = Router(
            dim,
            n_experts,
            top_k,
            bias_update_speed=bias_update_speed,
            route_scale=route_scale,
        )
        gate_EDM, up_EDM, down_EMD = _init_expert_weights(n_experts, dim, self.hidden_dim)
        self.w_gate_EDM = torch.nn.Parameter(gate_EDM)  # (E, D, M)
        self.w_up_EDM = torch.nn.Parameter(up_EDM)  # (E, D, M)
        self.w_down_EMD = torch.nn.Parameter(down_EMD)  # (E, M, D)

    def forward(self, x_BLD: torch.Tensor) -> torch.Tensor:
        return MoE.forward(self, x_BLD)
