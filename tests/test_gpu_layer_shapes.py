"""The MoE layer's forward and backward over a seeded sweep of shapes (moe.py:25-86 with the router of
router.py:40-70): expert counts 1..600, slots 1..min(E, 64), d_model and expert hidden sizes on and off
the kernels' 16-byte vector width (the module zero-pads the latter), batches 1..1500 tokens, bf16 and
fp32.  Each case: the output and every gradient against the oracle's autograd, judged as
test_gpu_moe.check_against does (within the contract tolerance of an fp64 evaluation, or no less
accurate than the reference's own computation in the layer's dtype), with the kernel's routing."""

import random

import pytest
import torch

from abacus.moe.moe import MoE
from test_gpu_moe import check_against

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _shapes():
    rng = random.Random(4242)
    out = []
    for _ in range(16):
        E = rng.choice([1, 2, 5, 8, 16, 33, 64, 130, 256, 300, 600])
        K = rng.randint(1, min(E, 64))
        D = rng.choice([8, 24, 64, 72, 128, 136, 256, 20, 100])
        M = rng.choice([8, 40, 64, 128, 200, 264, 12, 90])
        T = rng.choice([1, 7, 64, 300, 1000, 1500])
        dtype = torch.bfloat16 if rng.random() < 0.6 else torch.float32
        out.append((T, D, M, E, K, dtype))
    return out


SHAPES = _shapes()


@pytest.mark.parametrize("T,D,M,E,K,dtype", SHAPES,
                         ids=[f"T{t}_D{d}_M{m}_E{e}_K{k}_{str(dt)[6:]}" for t, d, m, e, k, dt in SHAPES])
def test_layer_shape_sweep(T, D, M, E, K, dtype):
    print(f"\n[layer-sweep] T={T} D={D} M={M} E={E} K={K} {dtype}", flush=True)
    torch.manual_seed(T + 31 * D + 7 * M + E * 3 + K)
    moe = MoE(D, E, K, hidden_dim=M, route_scale=1.5)
    with torch.no_grad():
        for p in (moe.router.w_DE, moe.w_gate_EDM, moe.w_up_EDM, moe.w_down_EMD):
            p.normal_(0.0, 0.1)
        moe.router.expert_bias_E.normal_(0.0, 0.02)
    moe = moe.to(DEV, dtype)
    x = torch.randn(T, D, device=DEV).to(dtype)
    target = torch.randn(T, D, device=DEV).to(dtype)
    check_against(moe, x, target, torch.device("cpu"))
