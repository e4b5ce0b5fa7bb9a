"""Routing on selection values the data rarely produce (router.py:46-49), shared by the GPU
and host-build tests: torch.topk's order puts NaN above every number (the first NaN first),
then +inf, exact ties go to the lower expert, -inf last, and bias = -sigmoid(0) makes exact
zeros.  Zero router weights on half the experts and zero inputs on half the tokens make those
logits exactly 0 (score 0.5), so the bias alone orders them; the other experts and tokens get
random logits.  Indices and weights are compared bit-exact with the oracle given the
library's logits."""

from __future__ import annotations

import torch

from abacus.moe.router import Router
from oracle import moe_oracle as oracle

SPECIAL_CASES = [(16, 5, torch.float32), (80, 10, torch.bfloat16), (256, 16, torch.float32), (64, 8, torch.bfloat16),
                 # the wide router (more than 256 experts or 16 slots): logits pass + top-k pass
                 (40, 24, torch.bfloat16), (300, 20, torch.float32), (1024, 64, torch.bfloat16)]
# bf16 batches of at least 8192 tokens with 129 or more experts take the router with 64-token blocks
LARGE_BATCH_CASES = [(256, 8, 8200), (160, 16, 8192), (512, 8, 8250), (1024, 64, 8192)]


def check_special_selection(E: int, K: int, dtype: torch.dtype, device: torch.device, T: int = 200) -> None:
    gen = torch.Generator().manual_seed(E * 31 + K)
    D = 64
    router = Router(D, E, K, bias_update_speed=0.0, route_scale=1.25)
    choices = torch.tensor([float("nan"), float("inf"), float("-inf"), -0.5, 0.0, 0.25, 0.25, -1.0])
    bias = choices[torch.randint(0, len(choices), (E,), generator=gen)]
    bias[E // 2] = float("nan")  # at least one NaN past the first 64 experts' lane block when E > 64
    with torch.no_grad():
        router.w_DE.zero_()
        router.w_DE[:, : E // 2] = torch.randn(D, E // 2, generator=gen) * 0.1
        router.expert_bias_E.copy_(bias)
    router = router.to(device=device, dtype=dtype)
    x = torch.randn(T, D, generator=gen)
    x[: T // 2] = 0.0
    x = x.to(device=device, dtype=dtype)
    router.eval()
    with torch.no_grad():
        weights, indices = router(x)
    r = router.last_routing
    w_o, idx_o, _ = oracle.route(r.logits_TE.cpu(), router.expert_bias_E.cpu(), K, router.route_scale)
    assert torch.equal(indices.cpu(), idx_o)
    assert torch.equal(weights.cpu(), w_o)
    nan_experts = torch.nonzero(torch.isnan(bias)).reshape(-1)
    first = nan_experts[: min(K, nan_experts.numel())].tolist()
    assert indices[: T // 2, : len(first)].cpu().tolist() == [first] * (T // 2)  # NaNs first, in index order
