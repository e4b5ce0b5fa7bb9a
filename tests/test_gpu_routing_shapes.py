"""Routing parity over a seeded sweep of shapes (router.py:40-70, moe.py:72-77): expert counts 1..1024,
slots 1..min(E, 64), batches 1..~9000 tokens, bf16 and fp32, so that every router form is drawn (the
fused kernel with its small-batch slices, the logits pass + top-k pass past 256 experts or 16 slots,
the 64-token blocks from 8192 tokens) along with both dispatch forms (the scan fused into the gather,
and the separate scan).  Through the layer in train mode: indices, weights, per-expert counts,
offsets, the permutation, each slot's dispatched row and the bias step bit-exact against the oracle
given the kernel's logits, and the logits close to an fp32 product of the same operands."""

import random

import numpy as np
import pytest
import torch

from abacus.moe.moe import MoE
from oracle import moe_oracle as oracle

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _shapes():
    rng = random.Random(20261202)
    out = []
    for i in range(24):
        E = rng.choice([1, 2, 3, 8, 17, 64, 100, 128, 129, 200, 256, 257, 384, 512, 640, 1024])
        K = rng.randint(1, min(E, 64))
        if i % 3 == 0:
            K = min(K, 16)  # the fused router's slot range, drawn more often
        T = rng.choice([1, 5, 16, 17, 300, 1024, 1025, 4000, 8192, 8250])
        D = 8 * rng.randint(1, 40)
        dtype = torch.bfloat16 if rng.random() < 0.7 else torch.float32
        out.append((T, D, E, K, dtype))
    return out


# and one of each router form for certain: the 64-token blocks (fused, 129..256 experts; and the
# logits pass beyond 256), the small-batch slices up to 64 and up to 256 experts, the fp32 fused form
SHAPES = _shapes() + [(8250, 64, 200, 8, torch.bfloat16), (8192, 128, 256, 16, torch.bfloat16),
                      (9000, 48, 1024, 8, torch.bfloat16), (700, 256, 64, 6, torch.bfloat16),
                      (300, 520, 160, 6, torch.bfloat16), (2000, 136, 48, 4, torch.float32)]


@pytest.mark.parametrize("T,D,E,K,dtype", SHAPES,
                         ids=[f"T{t}_D{d}_E{e}_K{k}_{str(dt)[6:]}" for t, d, e, k, dt in SHAPES])
def test_routing_shape_sweep(T, D, E, K, dtype):
    print(f"\n[routing-sweep] T={T} D={D} E={E} K={K} {dtype}", flush=True)
    torch.manual_seed(T * 131 + E * 7 + K)
    moe = MoE(D, E, K, hidden_dim=8, bias_update_speed=0.01, route_scale=1.25)
    with torch.no_grad():
        moe.router.w_DE.normal_(0.0, 0.5)
        moe.router.expert_bias_E.normal_(0.0, 0.05)
    moe = moe.to(DEV, dtype)
    x = torch.randn(T, D, device=DEV).to(dtype)
    bias0 = moe.router.expert_bias_E.detach().clone()
    moe.train()
    with torch.no_grad():
        moe(x)
    torch.cuda.synchronize()
    r = moe.router.last_routing
    w_o, idx_o, _ = oracle.route(r.logits_TE.cpu(), bias0.cpu(), K, moe.router.route_scale)
    assert torch.equal(r.indices_TK.cpu(), idx_o)
    assert torch.equal(r.weights_TK.cpu(), w_o)
    counts, offsets, perm, pos = oracle.dispatch(idx_o, E)
    assert np.array_equal(r.counts_E.cpu().numpy(), counts)
    assert np.array_equal(r.offsets_E1.cpu().numpy(), offsets)
    assert np.array_equal(r.perm_R.cpu().numpy(), perm)
    assert np.array_equal(r.pos_TK.cpu().numpy().reshape(-1), np.asarray(pos).reshape(-1))
    assert torch.equal(moe.router.expert_bias_E.cpu(), oracle.bias_step(bias0.cpu(), idx_o, E, moe.router.bias_update_speed))
    # the logits are an fp32-accumulated product of the same operands
    ref = x.float() @ moe.router.w_DE.float()
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    torch.testing.assert_close(r.logits_TE.float(), ref, rtol=tol, atol=tol * max(float(ref.abs().max()), 1e-6))
