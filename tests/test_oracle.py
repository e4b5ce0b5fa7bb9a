"""Pins the oracle (oracle/moe_oracle.py) against known answers, libraries and closed forms.

Nothing here retypes the oracle's formulas: each check compares it with a value
fixed independently (hard-coded known answers from the reference's own test,
torch built-ins, plain-Python fp64 math, brute force, finite differences).
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import moe_oracle as oracle


def _dense_swiglu_linear(x, w_gate_DM, w_up_DM, w_down_MD):
    """SwiGLU built from torch.nn.Linear layers (the reference's MLP test, tests/test_mlp.py:6-22)."""
    dim, hidden = w_gate_DM.shape
    gate = torch.nn.Linear(dim, hidden, bias=False, dtype=x.dtype)
    up = torch.nn.Linear(dim, hidden, bias=False, dtype=x.dtype)
    down = torch.nn.Linear(hidden, dim, bias=False, dtype=x.dtype)
    with torch.no_grad():
        gate.weight.copy_(w_gate_DM.T)
        up.weight.copy_(w_up_DM.T)
        down.weight.copy_(w_down_MD.T)
    return down(torch.nn.functional.silu(gate(x)) * up(x))


def test_router_known_answer():
    """The reference's router test (tests/test_moe.py:9-39): indices, weights and the bias step."""
    w_DE = torch.tensor([[2.0, 0.0, -2.0, 1.0]])
    bias = torch.tensor([0.0, 0.0, 10.0, 0.0])
    x = torch.ones(4, 1)
    logits = x @ w_DE
    weights, indices, _ = oracle.route(logits, bias, top_k=2, route_scale=2.5)
    # Expert 2 wins slot 0 only because of the bias; expert 0 has the next largest score.
    assert indices.tolist() == [[2, 0]] * 4
    s = [oracle.sigmoid_reference_scalar(v) for v in (2.0, 0.0, -2.0, 1.0)]
    expected_w = [2.5 * s[2] / (s[2] + s[0]), 2.5 * s[0] / (s[2] + s[0])]
    torch.testing.assert_close(weights, torch.tensor([expected_w] * 4), rtol=1e-6, atol=1e-7)
    stepped = oracle.bias_step(bias, indices, n_experts=4, speed=10.0)
    assert stepped.tolist() == [-10.0, 10.0, 0.0, 10.0]
    _, indices_next, _ = oracle.route(logits, stepped, top_k=2, route_scale=2.5)
    assert indices_next.tolist() == [[3, 1]] * 4


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_bias_step_rounding(dtype):
    """b += speed * sign(R - E*c) with both roundings in the bias dtype."""
    bias = torch.tensor([0.1, -0.3, 0.7, 0.0], dtype=dtype)
    indices = torch.tensor([[0, 1], [0, 2], [0, 1]])  # counts 3, 2, 1, 0; R = 6, E = 4
    stepped = oracle.bias_step(bias, indices, 4, 1e-3)
    signs = [-1.0, -1.0, 1.0, 1.0]  # 6 - 4*[3, 2, 1, 0] = [-6, -2, 2, 6]
    for i, sgn in enumerate(signs):
        inc = torch.tensor(1e-3 * sgn, dtype=torch.float32).to(dtype)
        want = (bias[i].float() + inc.float()).to(dtype)
        assert stepped[i].item() == want.item()
    assert torch.equal(oracle.bias_step(bias, indices, 4, 0.0), bias)


def test_sigmoid_cr_matches_fp64_scalar():
    vals = [0.0, 1e-8, -1e-8, 0.5, -0.5, 3.0, -3.0, 17.0, -17.0, 88.0, -88.0, 103.0, -103.0]
    gen = torch.Generator().manual_seed(0)
    vals += (torch.randn(2000, generator=gen) * 4).tolist()
    x = torch.tensor(vals, dtype=torch.float32)
    got = oracle.sigmoid_cr(x)
    want = torch.tensor([oracle.sigmoid_reference_scalar(v) for v in x.tolist()], dtype=torch.float64).to(torch.float32)
    assert torch.equal(got, want)


# torch's CPU fp32 sigmoid is not correctly rounded (about a third of values are 1 ulp
# off, a few 2 ulp); after rounding to bf16 the two agree almost everywhere.
@pytest.mark.parametrize("dtype,max_ulp,min_agree", [(torch.float32, 2, 0.6), (torch.bfloat16, 1, 0.99)])
def test_sigmoid_cr_close_to_torch(dtype, max_ulp, min_agree):
    gen = torch.Generator().manual_seed(1)
    x = (torch.randn(200_000, generator=gen) * 3).to(dtype)
    a = oracle.sigmoid_cr(x)
    b = torch.sigmoid(x)
    ibits = torch.int32 if dtype == torch.float32 else torch.int16
    # sigmoid is positive, so the bit patterns order like the values: ulp distance = bit distance
    dist = (a.view(ibits).to(torch.int64) - b.view(ibits).to(torch.int64)).abs()
    assert int(dist.max()) <= max_ulp
    assert float((a == b).float().mean()) > min_agree


def test_topk_canonical_matches_torch_without_ties():
    gen = torch.Generator().manual_seed(2)
    sel = torch.rand(4096, 64, generator=gen)
    k = 6
    got = oracle.topk_canonical(sel, k)
    want = torch.topk(sel, k, dim=-1).indices
    s = torch.sort(sel, dim=-1, descending=True).values
    tie_free = (s[:, : k + 1].diff(dim=-1) != 0).all(dim=-1)
    assert tie_free.float().mean() > 0.99
    assert torch.equal(got[tie_free], want[tie_free])


def test_topk_canonical_tie_rule_bruteforce():
    gen = torch.Generator().manual_seed(3)
    sel = torch.randint(0, 4, (500, 8), generator=gen).float() / 4  # heavy ties
    sel[0, 3] = float("nan")
    got = oracle.topk_canonical(sel, 3)
    for r in range(sel.shape[0]):
        row = sel[r].tolist()
        key = sorted(range(8), key=lambda e: (0 if math.isnan(row[e]) else 1, -(0 if math.isnan(row[e]) else row[e]), e))
        assert got[r].tolist() == key[:3]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_sum_in_pick_order(dtype):
    """The renormalisation denominator: a per-step-rounded Python loop (fp32 accumulation, one
    rounding to the dtype) on small rows; torch.sum equal where it adds left to right (K = 1-4
    and 8 on the CPU) and within 2(K-1) ulp of the sum for every K."""
    gen = torch.Generator().manual_seed(5)
    for K in range(1, 17):
        picked = torch.rand(300, K, generator=gen).to(dtype)
        got = oracle.sum_in_pick_order(picked)
        assert got.shape == (300, 1) and got.dtype == dtype
        for r in range(20):
            acc = np.float32(0.0)
            for v in picked[r].float().tolist():
                acc = np.float32(acc + np.float32(v))
            assert float(got[r, 0]) == float(torch.tensor(float(acc)).to(dtype)), (K, r)
        want = picked.sum(dim=-1, keepdim=True)
        if K in (1, 2, 3, 4, 8):
            assert torch.equal(got, want), K
        u = 2.0 ** -24 if dtype == torch.float32 else 2.0 ** -8
        tol = (2 * max(K - 1, 0) * 2.0 ** -24 + 2 * u) * want.double().abs()
        assert bool(((got.double() - want.double()).abs() <= tol).all()), K


def test_dispatch_matches_bruteforce_and_stable_argsort():
    gen = torch.Generator().manual_seed(4)
    for T, E, K in [(1, 4, 1), (7, 4, 2), (33, 8, 3), (64, 16, 6)]:
        idx = torch.stack([torch.randperm(E, generator=gen)[:K] for _ in range(T)])
        fast = oracle.dispatch(idx, E)
        slow = oracle.dispatch_bruteforce(idx, E)
        for a, b in zip(fast, slow):
            assert np.array_equal(a, b)
        order = torch.argsort(idx.reshape(-1), stable=True)
        assert np.array_equal(fast[2], (order // K).numpy())


def test_one_expert_matches_dense_mlp():
    """E = 1, K = 1 reduces to the dense SwiGLU (tests/test_moe.py:42-53, tests/test_mlp.py:6-22)."""
    torch.manual_seed(0)
    D, M = 4, 8
    x = torch.randn(6, D)
    w_DE = torch.randn(D, 1)
    wg, wu, wd = torch.randn(1, D, M), torch.randn(1, D, M), torch.randn(1, M, D)
    out, idx = oracle.moe_forward(x, w_DE, torch.zeros(1), wg, wu, wd, top_k=1)
    assert idx.eq(0).all()
    torch.testing.assert_close(out, _dense_swiglu_linear(x, wg[0], wu[0], wd[0]))


def test_forced_routing_all_tokens_to_expert_zero():
    """w_DE = -8 except column 0 = +8 (tests/test_moe_ep.py:94-102): every token on expert 0."""
    torch.manual_seed(2)
    D, E, M = 4, 4, 8
    x = torch.randn(6, D).abs() + 0.1
    w_DE = torch.full((D, E), -8.0)
    w_DE[:, 0] = 8.0
    wg, wu, wd = torch.randn(E, D, M), torch.randn(E, D, M), torch.randn(E, M, D)
    out, idx = oracle.moe_forward(x, w_DE, torch.zeros(E), wg, wu, wd, top_k=1)
    counts, offsets, perm, _ = oracle.dispatch(idx, E)
    assert counts.tolist() == [6, 0, 0, 0] and offsets.tolist() == [0, 6, 6, 6, 6]
    assert perm.tolist() == list(range(6))
    torch.testing.assert_close(out, _dense_swiglu_linear(x, wg[0], wu[0], wd[0]))


def _tiny_problem(seed=5, T=16, D=8, E=4, K=2, M=16, dtype=torch.float64):
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(T, D, generator=gen, dtype=dtype)
    w_DE = torch.randn(D, E, generator=gen, dtype=dtype) * 0.5
    wg = torch.randn(E, D, M, generator=gen, dtype=dtype) * 0.3
    wu = torch.randn(E, D, M, generator=gen, dtype=dtype) * 0.3
    wd = torch.randn(E, M, D, generator=gen, dtype=dtype) * 0.3
    return x, w_DE, wg, wu, wd


def test_closed_form_backward_matches_autograd():
    x, w_DE, wg, wu, wd = _tiny_problem()
    params = [t.clone().requires_grad_() for t in (x, w_DE, wg, wu, wd)]
    out, idx = oracle.moe_forward(params[0], params[1], torch.zeros(4, dtype=torch.float64), *params[2:], top_k=2,
                                  route_scale=1.5)
    dout = torch.randn(out.shape, generator=torch.Generator().manual_seed(6), dtype=torch.float64)
    out.backward(dout)
    closed = oracle.closed_form_backward(x, w_DE, wg, wu, wd, idx, dout, route_scale=1.5)
    for got, want in zip([p.grad for p in params], closed):
        np.testing.assert_allclose(got.numpy(), want, rtol=1e-9, atol=1e-11)


def test_gradcheck_fixed_routing():
    x, w_DE, wg, wu, wd = _tiny_problem(T=6, D=4, E=3, K=2, M=5)
    _, idx = oracle.moe_forward(x, w_DE, torch.zeros(3, dtype=torch.float64), wg, wu, wd, top_k=2)
    bias = torch.zeros(3, dtype=torch.float64)

    def f(*ts):
        return oracle.moe_forward(ts[0], ts[1], bias, *ts[2:], top_k=2, route_scale=1.5, indices_TK=idx)[0]

    inputs = [t.clone().requires_grad_() for t in (x, w_DE, wg, wu, wd)]
    assert torch.autograd.gradcheck(f, inputs, eps=1e-6, atol=1e-7)


def test_empty_tokens_returns_input():
    x = torch.zeros(0, 4)
    out, _ = oracle.moe_forward(x, torch.zeros(4, 2), torch.zeros(2), torch.zeros(2, 4, 3), torch.zeros(2, 4, 3),
                                torch.zeros(2, 3, 4), top_k=1)
    assert out is x


# ---------------------------------------------------------------------------
# load_balancing.py:8-41
# ---------------------------------------------------------------------------
def test_load_balancing_uniform_routing_is_coeff():
    # every expert gets 1/E of the slots and 1/E of the probability: sum(f p) = 1/E, times coeff * E
    E = 8
    probs = torch.full((E * 3, E), 1.0 / E)
    idx = torch.arange(E * 3).remainder(E).unsqueeze(1)
    loss = oracle.load_balancing_loss(probs, idx, coeff=0.03)
    assert abs(float(loss) - 0.03) < 1e-7


def test_load_balancing_collapsed_routing_is_coeff_times_e():
    E = 6
    probs = torch.zeros(10, E)
    probs[:, 0] = 1.0
    idx = torch.zeros(10, 2, dtype=torch.long)  # both slots repeat expert 0: counted once per token
    loss = oracle.load_balancing_loss(probs, idx, coeff=0.01)
    # f_0 = 10 / (10 * 2) = 0.5 (one count per token, K = 2), p_0 = 1
    assert abs(float(loss) - 0.5 * 1.0 * 0.01 * E) < 1e-7


@pytest.mark.parametrize("T,E,K,seed", [(1, 1, 1, 0), (5, 4, 3, 1), (17, 8, 2, 2), (9, 5, 6, 3)])
def test_load_balancing_matches_bruteforce(T, E, K, seed):
    g = torch.Generator().manual_seed(seed)
    probs = torch.rand(T, E, generator=g, dtype=torch.float64)
    idx = torch.randint(0, E, (T, K), generator=g)  # repeats within a token are likely
    got = oracle.load_balancing_loss(probs.float(), idx, coeff=0.02)
    want = oracle.load_balancing_bruteforce(probs.float(), idx, 0.02)
    assert abs(float(got) - want) <= 1e-6 * max(abs(want), 1e-6)


def test_load_balancing_batch_dims_and_no_slot_dim():
    g = torch.Generator().manual_seed(4)
    probs = torch.rand(2, 3, 4, generator=g)
    idx = torch.randint(0, 4, (2, 3), generator=g)  # no expert-choice dimension: K = 1
    got = oracle.load_balancing_loss(probs, idx)
    want = oracle.load_balancing_bruteforce(probs, idx.unsqueeze(-1), 1e-2)
    assert abs(float(got) - want) <= 1e-6 * abs(want)


def test_load_balancing_gradient_closed_form():
    # d loss / d probs[t, e] = coeff * E * f_E[e] / T: read off load_balancing.py:38-40
    g = torch.Generator().manual_seed(5)
    T, E, K, coeff = 7, 5, 2, 0.04
    probs = torch.rand(T, E, generator=g).requires_grad_()
    idx = torch.randint(0, E, (T, K), generator=g)
    oracle.load_balancing_loss(probs, idx, coeff).backward()
    f = torch.zeros(E)
    for t in range(T):
        for e in set(idx[t].tolist()):
            f[e] += 1.0 / (T * K)
    want = (coeff * E * f / T).expand(T, E)
    torch.testing.assert_close(probs.grad, want, rtol=1e-6, atol=1e-9)


def test_load_balancing_errors_and_empty():
    with pytest.raises(ValueError, match="must include an expert dimension"):
        oracle.load_balancing_loss(torch.tensor(1.0), torch.tensor(0))
    with pytest.raises(ValueError, match="has no experts"):
        oracle.load_balancing_loss(torch.zeros(3, 0), torch.zeros(3, 1, dtype=torch.long))
    with pytest.raises(ValueError, match="does not match"):
        oracle.load_balancing_loss(torch.zeros(3, 4), torch.zeros(2, 1, dtype=torch.long))
    with pytest.raises(ValueError, match="expert-choice dimensions"):
        oracle.load_balancing_loss(torch.zeros(3, 4), torch.zeros(3, 1, 1, dtype=torch.long))
    with pytest.raises(RuntimeError, match="non-negative"):
        oracle.load_balancing_loss(torch.zeros(3, 4), torch.full((3, 1), -1))
    with pytest.raises(RuntimeError, match="smaller than num_classes"):
        oracle.load_balancing_loss(torch.zeros(3, 4), torch.full((3, 1), 4))
    z = oracle.load_balancing_loss(torch.zeros(0, 4, dtype=torch.bfloat16), torch.zeros(0, 2, dtype=torch.long))
    assert z.shape == () and z.dtype == torch.bfloat16 and float(z) == 0.0


def test_load_balancing_one_hot_agrees_with_scatter():
    # the restatement's scatter of ones equals the reference's one_hot(...).amax(dim=1)
    g = torch.Generator().manual_seed(6)
    idx = torch.randint(0, 7, (40, 5), generator=g)
    want = F.one_hot(idx, 7).amax(dim=1).float()
    got = torch.zeros(40, 7).scatter_(1, idx, 1.0)
    assert torch.equal(got, want)
