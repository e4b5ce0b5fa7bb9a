"""HIP-graph replay of the eval-mode MoE forward (abacus_amd.graphs.GraphedForward).

Every replay is checked bit for bit against an eager forward of the same input run just
before it (the kernels sum in fixed orders, so the two agree exactly), over several
replays with other inputs and eager work in between: small batches (split router,
thin expert tiles), fp32, and larger batches whose down projection runs its split tail."""

import pytest
import torch

from abacus_amd import workloads as W
from abacus_amd.graphs import GraphedForward

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)

CASES = [W.SKEW_BF16_T64, W.TINY_F32, W.MID_F32.with_tokens(1, 2048), W.MIXTRAL_BF16.with_tokens(1, 1024)]


@pytest.mark.parametrize("wl", CASES, ids=[w.name for w in CASES])
def test_graph_replays_match_eager(wl):
    print(f"\n[graph] {wl.name} T={wl.tokens} D={wl.dim} E={wl.n_experts} K={wl.top_k}", flush=True)
    moe, x, _ = W.build_on_device(wl, DEV) if wl.dim >= 2048 else W.build(wl, device=DEV)
    moe.eval()
    g = GraphedForward(moe, x)
    gen = torch.Generator(device=DEV).manual_seed(5)
    inputs = [x] + [torch.randn(x.shape, generator=gen, device=DEV).to(x.dtype) for _ in range(2)]
    for rep in range(3):
        for i, xi in enumerate(inputs):
            with torch.no_grad():
                want = moe(xi).clone()
            idx_eager = moe.router.last_routing.indices_TK.clone()
            counts_eager = moe.router.last_routing.counts_E.clone()
            torch.cuda.synchronize()
            got = g(xi).clone()
            torch.cuda.synchronize()
            assert torch.equal(got, want), f"replay {rep}, input {i}"
            assert torch.equal(g.routing.indices_TK, idx_eager) and torch.equal(g.routing.counts_E, counts_eager)


def test_graph_rejects_other_shapes_and_training_mode():
    moe, x, _ = W.build(W.TINY_F32, device=DEV)
    moe.eval()
    g = GraphedForward(moe, x)
    with pytest.raises(ValueError):
        g(x[:, :-1])
    moe.train()
    with pytest.raises(ValueError):
        GraphedForward(moe, x)
