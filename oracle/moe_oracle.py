"""Oracle: CPU restatement of abacus's MoE layer. TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module, and only to check results (or as the timed CPU baseline) -- never as
part of the product path.

It restates, in this project's own code, the algorithm of
  abacus/moe/router.py:40-70   (sigmoid router, selection bias, top-k, renormalise, bias step)
  abacus/moe/moe.py:60-86      (per-expert mask -> gather -> SwiGLU -> weighted scatter -> stack-sum)
  abacus/moe/load_balancing.py:8-41 (Switch-Transformer auxiliary loss)
with the same per-op rounding as torch on CPU in the activation dtype.

Pinning (tests/test_oracle.py):
  sigmoid_cr            - fp64 closed form vs math.exp; within 2 ulp (fp32) / 1 ulp (bf16)
                          of torch.sigmoid, which is itself not correctly rounded
  topk_canonical        - torch.topk on tie-free rows; brute-force ranking on tiny inputs
  sum_in_pick_order     - torch.sum: equal for K = 1-4 and 8, within 2(K-1) ulp otherwise;
                          a Python fp64 loop rounded per step on tiny inputs
  dispatch              - brute-force restatement of the expert loop; torch.argsort(stable)
  bias_step             - the reference's known-answer test (router.py test: [-10, 10, 0, 10])
  router_forward        - the reference's known-answer test (indices [2, .], then [3, 1])
  moe_forward           - E=1,K=1 equals a dense SwiGLU built from torch.nn.Linear;
                          forced routing (w_DE = +-8) equals expert 0's MLP
  moe backward          - fp64 torch.autograd.gradcheck; closed_form_backward (Appendix-A
                          formulas in numpy fp64) against autograd
  load_balancing_loss   - closed forms (uniform routing -> coeff; collapsed routing ->
                          coeff * E); Python-loop brute force in fp64 with repeated slots;
                          gradient = coeff * E * f_E / T per element against autograd
Parity pinned this way for every function above; nothing is left "unpinned".

Tie rule (the reference leaves it to torch.topk, whose order among equal values
is implementation-defined): descending selection value, ties -> lower expert
index, NaN above every number.

Sum order of the K picked scores (the reference leaves it to torch.sum, whose
order is implementation-defined for K >= 5): left to right in pick order, fp32
accumulation for 16-bit dtypes, one rounding (sum_in_pick_order).  Pinned
against torch.sum: equal for K = 1-4 and 8, within 2(K-1) ulp of the sum for
other K.
"""

from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F


# ---------------------------------------------------------------------------
# Router (router.py:45-51)
# ---------------------------------------------------------------------------
def sigmoid_cr(logits: torch.Tensor) -> torch.Tensor:
    """sigmoid evaluated in fp64, rounded to fp32, then to the logits' dtype (router.py:45).

    Correctly rounded to fp32 (fp64 carries ~2^-52 relative error); the bf16
    value is the round-to-nearest-even of that fp32, i.e. the reference's
    "compute in float, round to bf16" with a correctly rounded float.
    """
    l64 = logits.detach().to(torch.float64)
    s64 = 1.0 / (1.0 + torch.exp(-l64))
    if logits.dtype == torch.float64:
        return s64
    return s64.to(torch.float32).to(logits.dtype)


class _SigmoidCR(torch.autograd.Function):
    """sigmoid_cr forward; torch's sigmoid backward grad * s * (1 - s) in the output dtype."""

    @staticmethod
    def forward(ctx, logits):
        s = sigmoid_cr(logits)
        ctx.save_for_backward(s)
        return s

    @staticmethod
    def backward(ctx, grad):
        (s,) = ctx.saved_tensors
        return torch.ops.aten.sigmoid_backward(grad, s)


def selection(scores: torch.Tensor, bias_E: torch.Tensor) -> torch.Tensor:
    """scores + expert_bias_E in the activation dtype (router.py:47)."""
    return scores.detach() + bias_E


def topk_canonical(sel: torch.Tensor, k: int) -> torch.Tensor:
    """Indices of the k largest values per row, descending; ties -> lower index; NaN first."""
    v = sel.detach().to(torch.float64).cpu().numpy()  # exact for every float dtype
    n = v.shape[-1]
    flat = v.reshape(-1, n)
    nan = np.isnan(flat)
    val = np.where(nan, 0.0, flat)
    # np.lexsort: last key is primary; it is stable, so equal keys keep index order.
    order = np.lexsort((-val, ~nan), axis=-1)
    return torch.from_numpy(order[:, :k].astype(np.int64).reshape(*v.shape[:-1], k)).to(sel.device)


def route(logits: torch.Tensor, bias_E: torch.Tensor, top_k: int, route_scale: float):
    """Routing from given logits (the identical-logits contract).

    Returns (weights, indices, scores): weights in the logits' dtype with the
    reference's op-by-op rounding (gather, sum, divide, scale).
    """
    scores = sigmoid_cr(logits)
    indices = topk_canonical(selection(scores, bias_E), top_k)
    picked = scores.gather(dim=-1, index=indices)
    weights = picked / sum_in_pick_order(picked)
    weights = weights * route_scale
    return weights, indices, scores


def sum_in_pick_order(picked: torch.Tensor) -> torch.Tensor:
    """The renormalisation's denominator (router.py:49), keepdim: the K picked scores added left to
    right in pick order, in fp32 for 16-bit dtypes (torch's accumulation type there), rounded once
    to the dtype.  torch.sum's order over K terms is implementation-defined: on the CPU it adds
    1-4 and 8 terms left to right and 5-7 and 9 or more in another order, so for those K the
    reference's own results differ from run to run of the implementation by up to 2(K-1) ulp of
    the sum."""
    acc_dtype = torch.float32 if picked.dtype in (torch.bfloat16, torch.float16) else picked.dtype
    acc = picked[..., :1].to(acc_dtype)
    for k in range(1, picked.shape[-1]):
        acc = acc + picked[..., k:k + 1].to(acc_dtype)
    return acc.to(picked.dtype)


def bias_step(bias_E: torch.Tensor, indices: torch.Tensor, n_experts: int, speed: float) -> torch.Tensor:
    """New expert bias after one update (router.py:57-70); returns a new tensor."""
    if speed == 0:
        return bias_E.clone()
    counts = torch.bincount(indices.reshape(-1).cpu(), minlength=n_experts)
    violation = counts.sum() - counts * n_experts
    step = torch.sign(violation.to(dtype=bias_E.dtype))
    return bias_E.cpu() + speed * step


# ---------------------------------------------------------------------------
# Dispatch (moe.py:72-77)
# ---------------------------------------------------------------------------
def dispatch(indices_TK: torch.Tensor, n_experts: int):
    """Expert-major, ascending-token row order of the reference's expert loop.

    Returns numpy int64 arrays (counts_E, offsets_E1, perm_R, pos_TK):
    perm_R[r] = token of routed row r; pos_TK[t, k] = routed row of slot (t, k).
    """
    idx = indices_TK.reshape(indices_TK.shape[0], -1).numpy().astype(np.int64)
    T, K = idx.shape
    flat = idx.reshape(-1)
    counts = np.bincount(flat, minlength=n_experts).astype(np.int64)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    # A token picks distinct experts, so a stable sort of slot ids by expert keeps
    # ascending tokens inside each expert.
    order = np.argsort(flat, kind="stable")
    perm = order // K
    pos = np.empty(T * K, dtype=np.int64)
    pos[order] = np.arange(T * K)
    return counts, offsets, perm, pos.reshape(T, K)


def dispatch_bruteforce(indices_TK: torch.Tensor, n_experts: int):
    """The expert loop of moe.py:72-77 written out literally (tiny inputs only)."""
    idx = indices_TK.tolist()
    rows = []
    for expert in range(n_experts):
        for t, slots in enumerate(idx):
            if expert in slots:
                rows.append((t, slots.index(expert)))
    perm = np.array([t for t, _ in rows], dtype=np.int64)
    pos = np.zeros((len(idx), len(idx[0]) if idx else 0), dtype=np.int64)
    for r, (t, k) in enumerate(rows):
        pos[t, k] = r
    counts = np.array([sum(expert in s for s in idx) for expert in range(n_experts)], dtype=np.int64)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    return counts, offsets, perm, pos


# ---------------------------------------------------------------------------
# Full layer (moe.py:60-86) with autograd
# ---------------------------------------------------------------------------
def moe_forward(
    x_TD: torch.Tensor,
    w_DE: torch.Tensor,
    bias_E: torch.Tensor,
    w_gate_EDM: torch.Tensor,
    w_up_EDM: torch.Tensor,
    w_down_EMD: torch.Tensor,
    top_k: int,
    route_scale: float = 1.0,
    indices_TK: torch.Tensor | None = None,
):
    """Differentiable restatement of MoE.forward on CPU tensors.

    If ``indices_TK`` is given the routing is taken from it (to follow a
    routing decided elsewhere from identical logits); otherwise it is decided
    here from x @ w_DE.  Returns (out_TD, indices_TK).
    """
    n_experts = w_DE.shape[1]
    logits = x_TD @ w_DE
    scores = _SigmoidCR.apply(logits)
    if indices_TK is None:
        indices_TK = topk_canonical(selection(scores, bias_E), top_k)
    picked = scores.gather(dim=-1, index=indices_TK)
    weights = picked / sum_in_pick_order(picked) * route_scale
    if x_TD.shape[0] == 0:
        return x_TD, indices_TK
    parts = []
    for expert in range(n_experts):
        chosen_TK = indices_TK == expert
        rows_T = chosen_TK.any(dim=-1)
        if not bool(rows_T.any()):
            continue
        xs = x_TD[rows_T]
        act = F.silu(xs @ w_gate_EDM[expert]) * (xs @ w_up_EDM[expert])
        ys = act @ w_down_EMD[expert]
        ws = (weights * chosen_TK).sum(dim=-1)[rows_T]
        part = x_TD.new_zeros(x_TD.shape)
        part[rows_T] = ys * ws.unsqueeze(-1)
        parts.append(part)
    return torch.stack(parts).sum(dim=0), indices_TK


# ---------------------------------------------------------------------------
# Closed-form backward (independent of autograd), numpy fp64
# ---------------------------------------------------------------------------
def closed_form_backward(x, w_DE, w_gate, w_up, w_down, indices, dout, route_scale=1.0):
    """Gradients of sum(out * dout) by the hand-derived formulas, in fp64.

    For token t, slot k, e = idx[t,k], rho = route_scale:
      s = sigmoid(x W_DE); w_k = rho s_k / S, S = sum_k s_k
      g = x Wg[e]; u = x Wu[e]; h = silu(g) u; y = h Wd[e]; out = sum_k w_k y_k
      dy_k = w_k dout;  dw_k = <dout, y_k>
      dh = dy Wd^T;  dWd[e] += h^T dy
      dg = dh u silu'(g);  du = dh silu(g);  dWg[e] += x^T dg;  dWu[e] += x^T du
      dx += dg Wg^T + du Wu^T
      ds_j = (rho dw_j - sum_k dw_k w_k) / S;  dl_j = ds_j s_j (1 - s_j)
      dx += dl W_DE^T;  dW_DE += x^T dl
    """
    x = np.asarray(x, np.float64)
    w_DE = np.asarray(w_DE, np.float64)
    wg = np.asarray(w_gate, np.float64)
    wu = np.asarray(w_up, np.float64)
    wd = np.asarray(w_down, np.float64)
    idx = np.asarray(indices, np.int64)
    dout = np.asarray(dout, np.float64)
    T, _ = x.shape
    K = idx.shape[1]
    s_full = 1.0 / (1.0 + np.exp(-(x @ w_DE)))
    s = np.take_along_axis(s_full, idx, axis=1)
    S = s.sum(axis=1, keepdims=True)
    w = route_scale * s / S
    dx = np.zeros_like(x)
    dWg, dWu, dWd = np.zeros_like(wg), np.zeros_like(wu), np.zeros_like(wd)
    dl = np.zeros((T, w_DE.shape[1]))
    dw = np.zeros((T, K))
    for t in range(T):
        for k in range(K):
            e = idx[t, k]
            g = x[t] @ wg[e]
            u = x[t] @ wu[e]
            sig = 1.0 / (1.0 + np.exp(-g))
            silu = g * sig
            h = silu * u
            y = h @ wd[e]
            dw[t, k] = dout[t] @ y
            dy = w[t, k] * dout[t]
            dh = wd[e] @ dy
            dWd[e] += np.outer(h, dy)
            dg = dh * u * (sig * (1.0 + g * (1.0 - sig)))
            du = dh * silu
            dWg[e] += np.outer(x[t], dg)
            dWu[e] += np.outer(x[t], du)
            dx[t] += wg[e] @ dg + wu[e] @ du
        c = (dw[t] * w[t]).sum()
        for k in range(K):
            ds = (route_scale * dw[t, k] - c) / S[t, 0]
            dl[t, idx[t, k]] += ds * s[t, k] * (1.0 - s[t, k])
    dx += dl @ w_DE.T
    dW_DE = x.T @ dl
    return dx, dW_DE, dWg, dWu, dWd


def sigmoid_reference_scalar(v: float) -> float:
    """Plain-Python fp64 logistic function (independent pin for sigmoid_cr)."""
    if v >= 0:
        return 1.0 / (1.0 + math.exp(-v))
    z = math.exp(v)
    return z / (1.0 + z)


# ---------------------------------------------------------------------------
# Switch-Transformer auxiliary loss (load_balancing.py:8-41)
# ---------------------------------------------------------------------------
def load_balancing_loss(router_probs: torch.Tensor, expert_indices: torch.Tensor, coeff: float = 1e-2):
    """Restatement of load_balancing.py:8-41 on CPU tensors; differentiable in router_probs.

    f_E: fraction of (token, slot) pairs per expert with each expert counted at
    most once per token (the reference's one_hot(...).amax(dim=1), here a scatter
    of ones); p_E: mean probability per expert in fp32; loss = sum(f_E * p_E) *
    (coeff * E), returned in router_probs' dtype.
    """
    if router_probs.ndim < 1:  # load_balancing.py:14-15
        raise ValueError("router_probs must include an expert dimension")
    n_experts = router_probs.shape[-1]
    if n_experts < 1:  # :17-18
        raise ValueError(f"router_probs has no experts, got shape {tuple(router_probs.shape)}")
    batch = router_probs.shape[:-1]
    if expert_indices.shape[: len(batch)] != batch:  # :20-24
        raise ValueError(
            f"expert_indices shape {tuple(expert_indices.shape)} does not match "
            f"router_probs batch {tuple(batch)}"
        )
    extra = expert_indices.ndim - len(batch)
    if extra > 1:  # :26-29
        raise ValueError(f"expert_indices has {extra} expert-choice dimensions, expected 0 or 1")
    probs_TE = router_probs.reshape(-1, n_experts).float()  # :30
    tokens = probs_TE.shape[0]
    if tokens == 0:  # :32-33
        return router_probs.new_zeros(())
    slots_TK = expert_indices.reshape(tokens, -1).to(dtype=torch.long)  # :34
    # torch.nn.functional.one_hot's own argument checks (:36)
    if slots_TK.numel() > 0:
        if int(slots_TK.min()) < 0:
            raise RuntimeError("Class values must be non-negative.")
        if int(slots_TK.max()) >= n_experts:
            raise RuntimeError("Class values must be smaller than num_classes.")
    k = slots_TK.shape[-1]
    if k == 0:  # amax over an empty slot dimension
        raise RuntimeError("amax(): Expected reduction dim 1 to have non-zero size.")
    dispatch_TE = torch.zeros(tokens, n_experts, dtype=torch.float32).scatter_(1, slots_TK, 1.0)  # :36
    f_E = dispatch_TE.sum(dim=0) / (tokens * k)  # :38
    p_E = probs_TE.sum(dim=0) / tokens  # :39
    loss = torch.sum(f_E * p_E) * (coeff * n_experts)  # :40
    return loss.to(dtype=router_probs.dtype)  # :41


def load_balancing_bruteforce(probs, indices, coeff):
    """Python-loop restatement in fp64 (tiny inputs): the definition read off load_balancing.py:36-40."""
    P = [[float(v) for v in row] for row in probs.reshape(-1, probs.shape[-1]).tolist()]
    T, E = len(P), probs.shape[-1]
    S = indices.reshape(T, -1).tolist()
    K = len(S[0])
    f = [0.0] * E
    for t in range(T):
        for e in set(S[t]):
            f[e] += 1.0
    f = [c / (T * K) for c in f]
    p = [sum(P[t][e] for t in range(T)) / T for e in range(E)]
    return sum(f[e] * p[e] for e in range(E)) * coeff * E
