"""The torch.topk comparison of tests/routing_check.py on the CPU: planted disagreements are
caught, ties and boundary sigmoid differences are the only exemptions, and on the synthetic
router inputs the exempt share equals the share of boundary ties."""

import pytest
import torch

from abacus_amd import workloads as W
from oracle import moe_oracle as oracle
from routing_check import check_against_torch_topk


def _route(logits, bias, k):
    _, idx, scores = oracle.route(logits, bias, k, 1.0)
    return idx, scores


def test_agrees_without_ties():
    torch.manual_seed(0)
    logits = torch.randn(300, 16)
    bias = torch.zeros(16)
    idx, scores = _route(logits, bias, 3)
    c = check_against_torch_topk(logits, bias, idx, scores)
    assert (c.ties, c.sigmoid_exempt, c.set_mismatches, c.invalid_exempt) == (0, 0, 0, 0)


def test_planted_wrong_set_is_a_mismatch():
    torch.manual_seed(1)
    logits = torch.randn(50, 8)
    bias = torch.zeros(8)
    idx, scores = _route(logits, bias, 2)
    bad = idx.clone()
    # token 7: swap its second pick for its lowest-ranked expert
    bad[7, 1] = int(torch.argsort(logits[7])[0])
    c = check_against_torch_topk(logits, bias, bad, scores)
    assert c.set_mismatches == 1 and c.exempt == 0


def test_tie_is_exempt_but_must_be_valid():
    logits = torch.tensor([[2.0, 1.0, 1.0, -1.0], [3.0, 0.5, 0.5, 0.5]])
    bias = torch.zeros(4)
    idx, scores = _route(logits, bias, 2)
    c = check_against_torch_topk(logits, bias, idx, scores)
    assert c.ties == 2 and c.set_mismatches == 0 and c.invalid_exempt == 0
    bad = torch.tensor([[0, 3], [0, 1]])  # expert 3 is below the tied pair on token 0
    c = check_against_torch_topk(logits, bias, bad, scores)
    assert c.ties == 2 and c.invalid_exempt == 1


def test_sigmoid_difference_at_the_boundary_is_exempt():
    # Kernel scores one ulp above torch's on expert 1 lift it over expert 2.
    logits = torch.tensor([[4.0, 0.3, 0.3000002, -2.0]])
    bias = torch.zeros(4)
    s_t = torch.sigmoid(logits)
    assert s_t[0, 1] < s_t[0, 2]  # one fp32 ulp apart
    scores = s_t.clone()
    scores[0, 1] = torch.nextafter(s_t[0, 2], torch.tensor(2.0))
    picked = torch.tensor([[0, 1]])
    c = check_against_torch_topk(logits, bias, picked, scores)
    assert c.sigmoid_exempt == 1 and c.set_mismatches == 0 and c.invalid_exempt == 0
    # Expert 3 is far below: picking it is invalid even with the difference.
    c = check_against_torch_topk(logits, bias, torch.tensor([[0, 3]]), scores)
    assert c.sigmoid_exempt == 1 and c.invalid_exempt == 1
    # The same difference far from the boundary exempts nothing.
    scores2 = s_t.clone()
    scores2[0, 0] = torch.nextafter(s_t[0, 0], torch.tensor(0.0))
    idx = torch.topk(s_t, 2, dim=-1).indices
    c = check_against_torch_topk(logits, bias, idx, scores2)
    assert c.exempt == 0 and c.set_mismatches == 0


@pytest.mark.parametrize("wl,tie_share", [(W.MIXTRAL_BF16, (0.005, 0.04)), (W.SKEW_BF16_T512, (0.05, 0.16)),
                                          (W.MID_F32, (0.0, 0.0))])
def test_exempt_share_is_the_tie_share(wl, tie_share):
    """Router logits of the workload's shape (1024 tokens): exemptions are ties only."""
    torch.manual_seed(wl.seed)
    T = 1024
    x = torch.randn(T, wl.dim).to(wl.dtype)
    w = (torch.randn(wl.dim, wl.n_experts) * 0.02).to(wl.dtype)
    bias = W.zipf_bias(wl.n_experts).to(wl.dtype) if wl.zipf_bias else torch.zeros(wl.n_experts, dtype=wl.dtype)
    logits = (x.float() @ w.float()).to(wl.dtype)
    idx, scores = _route(logits, bias, wl.top_k)
    c = check_against_torch_topk(logits, bias, idx, scores)
    print(c.summary())
    assert c.set_mismatches == 0 and c.invalid_exempt == 0
    assert tie_share[0] <= c.ties / T <= tie_share[1]
    assert c.sigmoid_exempt <= T // 100
