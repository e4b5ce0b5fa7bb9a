"""The MoE decoder that calls the MoE layer: TransformerMoe and its parts.

Single-GPU restatements of the reference's caller modules, with their
constructor signatures, parameter names and shapes, buffers and
initialisation RNG order, so a seeded model and its state_dict match the
reference's:

  Embedding            abacus/embedding.py:8-23
  Rotary, rotate_half,
  apply_rotary_pos_emb abacus/rope.py:9-46
  RMSNorm              abacus/norm.py:11-31
  MultiHeadAttention   abacus/attention.py:67-150, 188-218 (the single-rank path)
  TransformerBlockMoe  abacus/transformer_block.py:64-110
  TransformerMoe       abacus/transformer_moe.py:17-75

The MoE layer inside each block is abacus_amd.moe.MoE (the HIP path).  On
the GPU, RMSNorm, the q/k norms fused with the rotary embedding, and causal
attention in bf16 with head dim 64 (L a multiple of 128) also run on this
library's HIP kernels; the (L, L) scores never reach HBM and stay fp32 where
the reference rounds them to the activation dtype.  Other attention inputs go
to torch's fused causal kernels (flash / memory-efficient), and on the CPU,
or for inputs no fused kernel takes, attention is materialised like the
reference's (scores, mask, softmax, weighted sum) as one autograd function
whose batched products all take contiguous operands.  The dense projections
and the embedding run on torch.  Tensor, sequence and context parallelism
with more than one process are not implemented here (one GPU).
"""

from __future__ import annotations

import math

import torch

from . import _lib
from .moe import MoE, MoEExpertParallel, _rank_and_world_size

__all__ = [
    "Embedding",
    "Rotary",
    "rotate_half",
    "apply_rotary_pos_emb",
    "RMSNorm",
    "MultiHeadAttention",
    "TransformerBlockMoe",
    "TransformerMoe",
]


def _single_process(what: str) -> None:
    if _rank_and_world_size()[1] > 1:
        raise NotImplementedError(f"{what} across processes is not part of this single-GPU build")


class Embedding(torch.nn.Module):
    """Token embedding table (embedding.py:8-23): w_vocab_D ~ N(0, 1)."""

    def __init__(self, vocab_size: int, dim: int):
        super().__init__()
        self.vocab_size = vocab_size
        self.dim = dim
        self.w_vocab_D = torch.nn.Parameter(torch.empty(vocab_size, dim))
        torch.nn.init.normal_(self.w_vocab_D)

    def forward(self, tokens_BL: torch.Tensor) -> torch.Tensor:
        return self.w_vocab_D[tokens_BL]  # (B, L, D)


class Rotary(torch.nn.Module):
    """Rotary position tables (rope.py:9-32): cos/sin of position x inv_freq, cached per length.

    inv_freq is a buffer, so Module.to(dtype) casts it and the tables follow
    the model's dtype, as in the reference.
    """

    def __init__(self, dim: int, base: float = 10000):
        super().__init__()
        inv_freq = 1.0 / (base ** (torch.arange(0, dim, 2).float() / dim))  # (K / 2,)
        self.register_buffer("inv_freq", inv_freq)
        self.seq_len_cached = None
        self.cos_cached = None
        self.sin_cached = None

    def forward(self, x: torch.Tensor, seq_dim: int = 2, positions: torch.Tensor | None = None):
        if positions is not None:
            return self._angles(x, positions)
        seq_len = x.shape[seq_dim]
        if seq_len != self.seq_len_cached:
            self.seq_len_cached = seq_len
            self.cos_cached, self.sin_cached = self._angles(x, torch.arange(seq_len, device=x.device))
        return self.cos_cached, self.sin_cached  # (1, 1, L, K)

    def _angles(self, x: torch.Tensor, positions: torch.Tensor):
        t = positions.to(device=x.device).type_as(self.inv_freq)  # (L,)
        freqs = torch.outer(t, self.inv_freq)  # (L, K / 2)
        emb = torch.cat((freqs, freqs), dim=-1).to(x.device)  # (L, K)
        return emb.cos()[None, None, :, :], emb.sin()[None, None, :, :]


def rotate_half(x: torch.Tensor) -> torch.Tensor:
    """(x1, x2) -> (-x2, x1) over the last dimension's halves (rope.py:35-40)."""
    half = x.shape[-1] // 2
    return torch.cat((-x[..., half:], x[..., :half]), dim=-1)


def apply_rotary_pos_emb(q, k, cos, sin):
    """q cos + rotate_half(q) sin, likewise for k (rope.py:43-46)."""
    return (q * cos) + (rotate_half(q) * sin), (k * cos) + (rotate_half(k) * sin)


def _fused_norm_ok(x: torch.Tensor, gamma: torch.Tensor) -> bool:
    """The HIP RMSNorm takes x: GPU, fp32/bf16, gamma of the same dtype, and rows whose
    16-byte vectors split evenly over a power-of-two number of lanes (at most 8 each)."""
    if not (x.is_cuda and x.dtype in (torch.float32, torch.bfloat16) and gamma.dtype == x.dtype):
        return False
    D = x.shape[-1]
    epv = 8 if x.dtype == torch.bfloat16 else 4
    if D % epv:
        return False
    nvec, lpr = D // epv, 64
    while lpr > 1 and nvec % lpr:
        lpr //= 2
    return nvec // lpr in (1, 2, 4, 8)


class _RMSNormFunction(torch.autograd.Function):
    """gamma * x / sqrt(mean(x^2) + eps) as one HIP kernel each way (fp32 inside,
    one rounding per output; dgamma reduced in a fixed order)."""

    @staticmethod
    def forward(ctx, x, gamma, eps: float):
        D = x.shape[-1]
        xc = x.contiguous()
        rows = xc.numel() // D
        y = torch.empty_like(xc)
        rstd = torch.empty(rows, dtype=torch.float32, device=x.device)
        _lib.call("abacus_rmsnorm_fwd", _lib.ptr(xc), _lib.ptr(gamma.contiguous()), rows, D, eps,
                  _lib.dtype_code(x.dtype), _lib.ptr(y), _lib.ptr(rstd), _lib.stream_of(x.device))
        ctx.save_for_backward(xc, gamma, rstd)
        return y.view(x.shape)

    @staticmethod
    def backward(ctx, dy):
        xc, gamma, rstd = ctx.saved_tensors
        D = xc.shape[-1]
        rows = xc.numel() // D
        dyc = dy.contiguous()
        dx = torch.empty_like(xc)
        dgamma = torch.empty_like(gamma)
        nbytes = _lib.query("abacus_rmsnorm_bwd_ws_bytes", rows, D)
        ws = torch.empty(max(1, nbytes // 4), dtype=torch.float32, device=dy.device)
        _lib.call("abacus_rmsnorm_bwd", _lib.ptr(dyc), _lib.ptr(xc), _lib.ptr(gamma.contiguous()), _lib.ptr(rstd),
                  rows, D, _lib.dtype_code(xc.dtype), _lib.ptr(dx), _lib.ptr(dgamma), _lib.ptr(ws), nbytes,
                  _lib.stream_of(dy.device))
        return dx.view(dy.shape), dgamma, None


def _fused_rope_ok(x: torch.Tensor, gamma: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> bool:
    """The HIP norm + rotary kernel takes what the fused norm takes, with cos/sin of
    x's dtype and a row of 2..64 16-byte vectors, a power of two (one per lane)."""
    if not (_fused_norm_ok(x, gamma) and cos.dtype == x.dtype and sin.dtype == x.dtype):
        return False
    nvec = x.shape[-1] // (8 if x.dtype == torch.bfloat16 else 4)
    return 2 <= nvec <= 64 and nvec & (nvec - 1) == 0


class _RMSNormRopeFunction(torch.autograd.Function):
    """RMSNorm over K of a (B, L, H, K) tensor, then the rotary embedding at each
    row's position l: one HIP kernel each way."""

    @staticmethod
    def forward(ctx, x_BLHK, gamma, cos_LK, sin_LK, eps: float):
        B, L, H, K = x_BLHK.shape
        xc = x_BLHK.contiguous()
        rows = B * L * H
        y = torch.empty_like(xc)
        rstd = torch.empty(rows, dtype=torch.float32, device=xc.device)
        cos_c, sin_c = cos_LK.contiguous(), sin_LK.contiguous()
        _lib.call("abacus_rmsnorm_rope_fwd", _lib.ptr(xc), _lib.ptr(gamma.contiguous()), _lib.ptr(cos_c),
                  _lib.ptr(sin_c), rows, L, H, K, eps, _lib.dtype_code(xc.dtype), _lib.ptr(y), _lib.ptr(rstd),
                  _lib.stream_of(xc.device))
        ctx.save_for_backward(xc, gamma, rstd, cos_c, sin_c)
        return y

    @staticmethod
    def backward(ctx, dy):
        xc, gamma, rstd, cos_c, sin_c = ctx.saved_tensors
        B, L, H, K = xc.shape
        rows = B * L * H
        dyc = dy.contiguous()
        dx = torch.empty_like(xc)
        dgamma = torch.empty_like(gamma)
        nbytes = _lib.query("abacus_rmsnorm_bwd_ws_bytes", rows, K)
        ws = torch.empty(max(1, nbytes // 4), dtype=torch.float32, device=dy.device)
        _lib.call("abacus_rmsnorm_rope_bwd", _lib.ptr(dyc), _lib.ptr(xc), _lib.ptr(gamma.contiguous()),
                  _lib.ptr(rstd), _lib.ptr(cos_c), _lib.ptr(sin_c), rows, L, H, K, _lib.dtype_code(xc.dtype),
                  _lib.ptr(dx), _lib.ptr(dgamma), _lib.ptr(ws), nbytes, _lib.stream_of(dy.device))
        return dx, dgamma, None, None, None


class RMSNorm(torch.nn.Module):
    """gamma * x / sqrt(mean(x^2) + 1e-5) over the last dimension (norm.py:11-31).

    On the GPU one fused HIP kernel each way (``abacus_rmsnorm_fwd`` / ``_bwd``);
    on the CPU, or for inputs the kernel does not take, the reference's ops.
    """

    def __init__(self, dim: int, sequence_parallel: bool = False, sync_grads: bool = False):
        super().__init__()
        self.dim = dim
        self.sequence_parallel = sequence_parallel
        self.sync_grads = sequence_parallel or sync_grads
        self.world_size = _rank_and_world_size()[1] if self.sync_grads else 1
        self.w_gamma_D = torch.nn.Parameter(torch.ones(self.dim))

    def forward(self, x_BLD: torch.Tensor) -> torch.Tensor:
        if self.sync_grads and self.world_size > 1:
            _single_process("RMSNorm gradient synchronisation")
        if _fused_norm_ok(x_BLD, self.w_gamma_D):
            return _RMSNormFunction.apply(x_BLD, self.w_gamma_D, 1e-5)
        rms_BL = torch.sqrt(x_BLD.square().mean(dim=-1, keepdim=True) + 1e-5)  # (B, L, 1)
        return self.w_gamma_D * x_BLD / rms_BL


class _CausalAttention(torch.autograd.Function):
    """softmax(mask(q k^T / sqrt(K))) v over (B*H, L, K) blocks (attention.py:136-141).

    Forward and backward as four batched products whose operands are all
    contiguous; the softmax backward is torch's own kernel, so the gradients
    are the ones autograd would form from the same forward.
    """

    @staticmethod
    def forward(ctx, q, k, v, scale_div: float):
        BH, L, K = q.shape
        s = torch.bmm(q, k.transpose(1, 2).contiguous())  # (BH, L, L)
        s = s / scale_div
        later = torch.ones(L, L, dtype=torch.bool, device=q.device).triu_(1)  # key after its query
        s = s.masked_fill(later, float("-inf"))
        p = torch.softmax(s, dim=-1)
        out = torch.bmm(p, v)  # (BH, L, K)
        ctx.save_for_backward(q, k, v, p)
        ctx.scale_div = scale_div
        return out

    @staticmethod
    def backward(ctx, d_out):
        q, k, v, p = ctx.saved_tensors
        d_out = d_out.contiguous()
        d_p = torch.bmm(d_out, v.transpose(1, 2).contiguous())
        # dV = P^T dO and dK = dS^T q, formed as (dO^T P)^T and (q^T dS)^T: the
        # (L, L) matrices stay contiguous and only (L, K) operands are transposed
        d_v = torch.bmm(d_out.transpose(1, 2).contiguous(), p).transpose(1, 2)
        d_s = torch._softmax_backward_data(d_p, p, -1, p.dtype)  # zero where the mask put -inf
        d_s = d_s / ctx.scale_div
        d_q = torch.bmm(d_s, k)
        d_k = torch.bmm(q.transpose(1, 2).contiguous(), d_s).transpose(1, 2)
        return d_q, d_k, d_v, None


# Fused causal attention on the GPU: torch's flash / memory-efficient
# kernels (scores and probabilities stay on chip, in fp32), never its
# materializing math path.  Inputs neither kernel takes fall back to
# _CausalAttention; the outcome is kept per (dtype, head_dim).
_FUSED_BACKENDS = None
_fused_ok: dict = {}


def _fused_causal_attention(q, k, v):
    """softmax(mask(q k^T / sqrt(K))) v for (B, H, L, K) q, k, v, or None."""
    global _FUSED_BACKENDS
    key = (q.dtype, q.shape[-1])
    if _fused_ok.get(key) is False or not (q.dtype == k.dtype == v.dtype):
        return None
    try:
        from torch.nn.attention import SDPBackend, sdpa_kernel
    except ImportError:
        _fused_ok[key] = False
        return None
    if _FUSED_BACKENDS is None:
        _FUSED_BACKENDS = [SDPBackend.EFFICIENT_ATTENTION, SDPBackend.FLASH_ATTENTION]
    try:
        with sdpa_kernel(_FUSED_BACKENDS):
            out = torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=True)
    except RuntimeError:
        # no fused kernel for these inputs (raised before any launch)
        _fused_ok[key] = False
        return None
    _fused_ok[key] = True
    return out


def _flash_ok(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> bool:
    """abacus_attention_fwd takes contiguous bf16 (B, L, H, 64) q, k, v on the GPU, L a multiple of 128."""
    return (q.is_cuda and q.dim() == 4 and q.dtype == torch.bfloat16 and q.shape[-1] == 64 and q.shape[1] % 128 == 0
            and all(t.dtype == q.dtype and t.shape == q.shape and t.is_contiguous() for t in (q, k, v)))


class _FlashAttentionFunction(torch.autograd.Function):
    """Causal attention (attention.py:136-141) in the (B, L, H, K) layout by the HIP flash kernels.

    The forward keeps scores and probabilities on chip in fp32 and saves each
    query's log2-sum-exp2; the backward rebuilds the probabilities from it and
    forms dq, dk, dv without materialising an (L, L) matrix.
    """

    @staticmethod
    def forward(ctx, q_BLHK, k_BLHK, v_BLHK):
        B, L, H, K = q_BLHK.shape
        o = torch.empty_like(q_BLHK)
        lse = torch.empty(B, H, L, dtype=torch.float32, device=q_BLHK.device)
        _lib.call("abacus_attention_fwd", _lib.ptr(q_BLHK), _lib.ptr(k_BLHK), _lib.ptr(v_BLHK), B, L, H, K,
                  1.0 / math.sqrt(K), _lib.BF16, _lib.ptr(o), _lib.ptr(lse), _lib.stream_of(q_BLHK.device))
        ctx.save_for_backward(q_BLHK, k_BLHK, v_BLHK, o, lse)
        return o

    @staticmethod
    def backward(ctx, d_o):
        q, k, v, o, lse = ctx.saved_tensors
        B, L, H, K = q.shape
        d_o = d_o.contiguous()
        dq, dk, dv = (torch.empty_like(q) for _ in range(3))
        nbytes = _lib.query("abacus_attention_bwd_ws_bytes", B, L, H)
        ws = torch.empty(nbytes // 4, dtype=torch.float32, device=q.device)
        _lib.call("abacus_attention_bwd", _lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(o), _lib.ptr(d_o),
                  _lib.ptr(lse), B, L, H, K, 1.0 / math.sqrt(K), _lib.BF16, _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv),
                  _lib.ptr(ws), nbytes, _lib.stream_of(q.device))
        return dq, dk, dv


# The HIP flash kernels take the attention whenever _flash_ok holds; False
# sends it to torch's fused kernels (as for every other shape).
flash_attention_enabled = True


class _QKVProjection(torch.autograd.Function):
    """q, k, v = x W_q, x W_k, x W_v (attention.py:129-131) with one backward for the three.

    The forward runs the three products, each output contiguous as the
    kernels after it want. The backward concatenates dq, dk, dv once and
    forms dx = [dq dk dv] [W_q W_k W_v]^T and [dW_q dW_k dW_v] = x^T [dq dk dv]
    as two GEMMs over the joint width: at T = 8192, D = H*K = 1024 in bf16
    that takes 157 us against 249 us for three weight-gradient GEMMs (their
    1024-wide outputs leave hipBLASLt a single round of small tiles), three
    data-gradient GEMMs and two adds.
    """

    @staticmethod
    def forward(ctx, x_BLD, w_q_DHK, w_k_DHK, w_v_DHK):
        B, L, D = x_BLD.shape
        _, H, K = w_q_DHK.shape
        x_TD = x_BLD.reshape(B * L, D)
        outs = [(x_TD @ w.reshape(D, H * K)).view(B, L, H, K) for w in (w_q_DHK, w_k_DHK, w_v_DHK)]
        ctx.save_for_backward(x_TD, w_q_DHK, w_k_DHK, w_v_DHK)
        ctx.x_shape = (B, L, D)
        return tuple(outs)

    @staticmethod
    def backward(ctx, dq, dk, dv):
        x_TD, w_q, w_k, w_v = ctx.saved_tensors
        B, L, D = ctx.x_shape
        _, H, K = w_q.shape
        HK = H * K
        grads = [torch.zeros(B, L, H, K, dtype=x_TD.dtype, device=x_TD.device) if g is None else g
                 for g in (dq, dk, dv)]
        g_T3 = torch.cat([g.reshape(B * L, HK) for g in grads], dim=1)  # (T, 3HK)
        dx = dwq = dwk = dwv = None
        if ctx.needs_input_grad[0]:
            w_D3 = torch.cat([w.reshape(D, HK) for w in (w_q, w_k, w_v)], dim=1)
            dx = (g_T3 @ w_D3.t()).view(B, L, D)
        if any(ctx.needs_input_grad[1:]):
            dw_D3 = x_TD.t() @ g_T3
            dwq, dwk, dwv = (dw_D3[:, i * HK:(i + 1) * HK].contiguous().view(D, H, K) if ctx.needs_input_grad[1 + i]
                             else None for i in range(3))
        return dx, dwq, dwk, dwv


class MultiHeadAttention(torch.nn.Module):
    """Causal multi-head attention with QK-norm and RoPE (attention.py:67-150).

    Parameters w_q_DHK, w_k_DHK, w_v_DHK (D, H, K), w_o_HKD (H, K, D) drawn
    with xavier_uniform_ on their (D, H*K) / (H*K, D) views in that order,
    then q_norm and k_norm (RMSNorm over K).
    """

    def __init__(
        self,
        dim: int,
        n_heads: int,
        head_dim: int,
        tensor_parallel: bool = False,
        sequence_parallel: bool = False,
        context_parallel: bool = False,
    ):
        super().__init__()
        if sequence_parallel and not tensor_parallel:
            raise ValueError("sequence_parallel requires tensor_parallel")
        if context_parallel and (tensor_parallel or sequence_parallel):
            raise ValueError("context_parallel does not combine with tensor or sequence parallel")
        self.dim = dim
        self.n_heads = n_heads
        self.head_dim = head_dim
        self.tensor_parallel = tensor_parallel
        self.sequence_parallel = sequence_parallel
        self.context_parallel = context_parallel
        if tensor_parallel:
            self.rank, self.world_size = _rank_and_world_size()
            if n_heads % self.world_size != 0:
                raise ValueError(f"n_heads {n_heads} is not divisible by world size {self.world_size}")
        else:
            self.rank, self.world_size = 0, 1
        self.local_heads = n_heads // self.world_size
        q_DHK = torch.empty(dim, n_heads, head_dim)
        k_DHK = torch.empty(dim, n_heads, head_dim)
        v_DHK = torch.empty(dim, n_heads, head_dim)
        o_HKD = torch.empty(n_heads, head_dim, dim)
        for w in (q_DHK, k_DHK, v_DHK):
            torch.nn.init.xavier_uniform_(w.view(dim, n_heads * head_dim))
        torch.nn.init.xavier_uniform_(o_HKD.view(n_heads * head_dim, dim))
        h0, h1 = self.rank * self.local_heads, (self.rank + 1) * self.local_heads
        self.w_q_DHK = torch.nn.Parameter(q_DHK[:, h0:h1].clone())
        self.w_k_DHK = torch.nn.Parameter(k_DHK[:, h0:h1].clone())
        self.w_v_DHK = torch.nn.Parameter(v_DHK[:, h0:h1].clone())
        self.w_o_HKD = torch.nn.Parameter(o_HKD[h0:h1].clone())
        sync_qk = tensor_parallel or context_parallel
        self.q_norm = RMSNorm(head_dim, sync_grads=sync_qk)
        self.k_norm = RMSNorm(head_dim, sync_grads=sync_qk)

    def forward(self, x_BLD: torch.Tensor, rotary: Rotary | None = None) -> torch.Tensor:
        if self.context_parallel or self.world_size > 1:
            _single_process("attention parallelism")
        B, L, _ = x_BLD.shape
        H, K = self.local_heads, self.head_dim
        q_heads, k_heads, v_heads = _QKVProjection.apply(x_BLD, self.w_q_DHK, self.w_k_DHK, self.w_v_DHK)
        cos = sin = None
        if rotary is not None:
            cos, sin = rotary(q_heads, seq_dim=1)  # (1, 1, L, K)
        if (cos is not None and _fused_rope_ok(q_heads, self.q_norm.w_gamma_D, cos, sin)
                and _fused_rope_ok(k_heads, self.k_norm.w_gamma_D, cos, sin)):
            # q/k norm and the rotary embedding in one HIP kernel each
            cos_LK, sin_LK = cos.reshape(L, K), sin.reshape(L, K)
            q_blhk = _RMSNormRopeFunction.apply(q_heads, self.q_norm.w_gamma_D, cos_LK, sin_LK, 1e-5)
            k_blhk = _RMSNormRopeFunction.apply(k_heads, self.k_norm.w_gamma_D, cos_LK, sin_LK, 1e-5)
            if flash_attention_enabled and _flash_ok(q_blhk, k_blhk, v_heads):
                # the HIP flash kernels on the (B, L, H, K) layout: no permuted copies
                out = _FlashAttentionFunction.apply(q_blhk, k_blhk, v_heads)
                return out.reshape(B, L, H * K) @ self.w_o_HKD.reshape(H * K, self.dim)
            q, k = q_blhk.permute(0, 2, 1, 3), k_blhk.permute(0, 2, 1, 3)
        else:
            q = self.q_norm(q_heads).permute(0, 2, 1, 3)  # (B, H, L, K)
            k = self.k_norm(k_heads).permute(0, 2, 1, 3)
            if rotary is not None:
                q, k = apply_rotary_pos_emb(q, k, cos, sin)
        v = v_heads.permute(0, 2, 1, 3)  # (B, H, L, K)
        out = _fused_causal_attention(q, k, v) if q.is_cuda else None  # (B, H, L, K)
        if out is None:
            out = _CausalAttention.apply(
                q.reshape(B * H, L, K).contiguous(), k.reshape(B * H, L, K).contiguous(),
                v.reshape(B * H, L, K).contiguous(), self.head_dim ** 0.5,
            ).view(B, H, L, K)
        joined = out.permute(0, 2, 1, 3).reshape(B, L, H * K)
        return joined @ self.w_o_HKD.reshape(H * K, self.dim)  # (B, L, D)


class TransformerBlockMoe(torch.nn.Module):
    """x + attention(RMSNorm(x)), then x + MoE(RMSNorm(x)) (transformer_block.py:64-110)."""

    def __init__(
        self,
        dim: int,
        n_heads: int,
        head_dim: int,
        n_experts: int,
        top_k: int,
        dropout: float = 0.0,
        hidden_dim: int | None = None,
        bias_update_speed: float = 1e-3,
        route_scale: float = 1.0,
        expert_parallel: bool = False,
    ):
        super().__init__()
        _, world_size = _rank_and_world_size()
        if expert_parallel and dropout > 0 and world_size > 1:
            raise ValueError("expert parallel keeps dropout at 0 so replicated layers stay identical")
        self.dim = dim
        self.n_heads = n_heads
        self.head_dim = head_dim
        self.norm_attention = RMSNorm(dim)
        self.attention = MultiHeadAttention(dim, n_heads, head_dim)
        self.norm_mlp = RMSNorm(dim)
        moe = MoEExpertParallel if expert_parallel else MoE
        self.moe = moe(
            dim, n_experts, top_k, hidden_dim=hidden_dim, bias_update_speed=bias_update_speed,
            route_scale=route_scale,
        )
        self.dropout = torch.nn.Dropout(dropout)

    def forward(self, x_BLD: torch.Tensor, rotary: torch.nn.Module | None = None) -> torch.Tensor:
        attn_BLD = self.attention(self.norm_attention(x_BLD), rotary)
        x_BLD = x_BLD + self.dropout(attn_BLD)
        moe_BLD = self.moe(self.norm_mlp(x_BLD))
        return x_BLD + self.dropout(moe_BLD)


class TransformerMoe(torch.nn.Module):
    """Embedding -> n_blocks x TransformerBlockMoe -> RMSNorm -> logits (transformer_moe.py:17-75)."""

    def __init__(
        self,
        dim: int,
        n_heads: int,
        head_dim: int,
        n_blocks: int,
        vocab_size: int,
        n_experts: int,
        top_k: int,
        dropout: float = 0.0,
        hidden_dim: int | None = None,
        bias_update_speed: float = 1e-3,
        route_scale: float = 1.0,
        expert_parallel: bool = False,
    ):
        super().__init__()
        self.dim = dim
        self.n_heads = n_heads
        self.head_dim = head_dim
        self.n_blocks = n_blocks
        self.vocab_size = vocab_size
        self.n_experts = n_experts
        self.top_k = top_k
        self.expert_parallel = expert_parallel
        self.embedding = Embedding(vocab_size, dim)
        self.rotary = Rotary(head_dim)
        self.blocks = torch.nn.ModuleList(
            [
                TransformerBlockMoe(
                    dim, n_heads, head_dim, n_experts, top_k, dropout, hidden_dim=hidden_dim,
                    bias_update_speed=bias_update_speed, route_scale=route_scale, expert_parallel=expert_parallel,
                )
                for _ in range(n_blocks)
            ]
        )
        self.norm = RMSNorm(dim)
        self.w_D_vocab = torch.nn.Parameter(torch.empty(dim, vocab_size))  # (D, vocab)
        torch.nn.init.xavier_uniform_(self.w_D_vocab)

    def forward(self, tokens_BL: torch.Tensor) -> torch.Tensor:
        x_BLD = self.embedding(tokens_BL)
        for block in self.blocks:
            x_BLD = block(x_BLD, self.rotary)
        return self.norm(x_BLD) @ self.w_D_vocab  # (B, L, vocab)
