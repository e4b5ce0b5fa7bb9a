"""load_balancing_loss on the GPU (load_balancing.py:8-41) against the oracle's restatement."""

import pytest
import torch

from abacus.moe.load_balancing import load_balancing_loss
from oracle import moe_oracle as oracle

pytestmark = pytest.mark.gpu

CASES = [
    # (probability shape, index shape, E range, seed)
    ((64, 8), (64, 2), 1),
    ((3, 700, 16), (3, 700, 6), 2),        # batch dims, 2100 tokens: two blocks
    ((10000, 64), (10000, 8), 3),          # five blocks
    ((4, 9, 5), (4, 9), 4),                # no expert-choice dimension: K = 1
    ((257, 300), (257, 3), 5),             # E > 256: one column loop per thread
    ((40, 1000), (40, 12), 6),
    ((1, 1), (1, 1), 7),
]


def _inputs(pshape, ishape, dtype, seed, repeats=True):
    g = torch.Generator().manual_seed(seed)
    E = pshape[-1]
    probs = torch.rand(pshape, generator=g).to(dtype)
    idx = torch.randint(0, E, ishape, generator=g)
    if not repeats and len(ishape) == len(pshape):
        idx = torch.argsort(torch.rand(pshape, generator=g), dim=-1)[..., : ishape[-1]]
    return probs, idx


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
@pytest.mark.parametrize("pshape,ishape,seed", CASES, ids=[f"{c[0]}" for c in CASES])
def test_loss_and_grad_match_oracle(dtype, pshape, ishape, seed):
    coeff = 0.013
    for repeats in (True, False):
        probs, idx = _inputs(pshape, ishape, dtype, seed, repeats)
        p_ref = probs.clone().requires_grad_()
        want = oracle.load_balancing_loss(p_ref, idx, coeff)
        want.backward()
        p_gpu = probs.cuda().requires_grad_()
        got = load_balancing_loss(p_gpu, idx.cuda(), coeff)
        assert got.dtype == dtype and got.shape == ()
        got.backward()
        if dtype == torch.float32:
            torch.testing.assert_close(got.cpu(), want, rtol=1e-5, atol=1e-8)
            torch.testing.assert_close(p_gpu.grad.cpu(), p_ref.grad, rtol=1e-6, atol=1e-12)
        else:
            # both round the same fp32 value (summation order aside) to bf16: at most one bf16 ulp apart
            assert abs(float(got) - float(want)) <= 2 ** -7 * abs(float(want)) + 1e-12
            assert torch.equal(p_gpu.grad.cpu(), p_ref.grad)


def test_deterministic_and_index_errors():
    probs, idx = _inputs((5000, 32), (5000, 4), torch.float32, 8)
    p, i = probs.cuda(), idx.cuda()
    a, b = load_balancing_loss(p, i), load_balancing_loss(p, i)
    assert torch.equal(a, b)
    bad = i.clone()
    bad[1234, 2] = -3
    with pytest.raises(RuntimeError, match="non-negative"):
        load_balancing_loss(p, bad)
    bad = i.clone()
    bad[4999, 0] = 32
    with pytest.raises(RuntimeError, match="smaller than num_classes"):
        load_balancing_loss(p, bad)
    with pytest.raises(RuntimeError, match="non-zero size"):
        load_balancing_loss(p, i[:, :0])


def test_known_answers():
    E = 8
    probs = torch.full((E * 4, E), 1.0 / E, device="cuda")
    idx = torch.arange(E * 4, device="cuda").remainder(E).unsqueeze(1)
    assert abs(float(load_balancing_loss(probs, idx, coeff=0.05)) - 0.05) < 1e-7
    probs = torch.zeros(10, 6, device="cuda")
    probs[:, 0] = 1.0
    idx = torch.zeros(10, 2, dtype=torch.long, device="cuda")
    assert abs(float(load_balancing_loss(probs, idx, coeff=0.01)) - 0.5 * 0.01 * 6) < 1e-7
