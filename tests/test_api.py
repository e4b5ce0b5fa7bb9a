"""Host-side API of the drop-in modules (no GPU compute): constructors, parameter layout,
initialisation RNG order and error behaviour of abacus.moe.{moe,router,load_balancing}
(reference: abacus/moe/router.py:15-37, abacus/moe/moe.py:25-57, :92-128,
abacus/moe/load_balancing.py:14-33)."""

import pytest
import torch

from abacus.mlp import MLP
from abacus.moe.moe import MoE, MoEExpertParallel
from abacus.moe.router import Router
from oracle import moe_oracle as oracle


def test_parameter_layout_and_state_dict():
    moe = MoE(dim=16, n_experts=4, top_k=2, hidden_dim=24)
    shapes = {k: tuple(v.shape) for k, v in moe.state_dict().items()}
    assert shapes == {
        "router.w_DE": (16, 4),
        "router.expert_bias_E": (4,),
        "w_gate_EDM": (4, 16, 24),
        "w_up_EDM": (4, 16, 24),
        "w_down_EMD": (4, 24, 16),
    }
    assert [n for n, _ in moe.named_parameters()] == ["w_gate_EDM", "w_up_EDM", "w_down_EMD", "router.w_DE"]
    assert moe.hidden_dim == 24 and MoE(8, 2, 1).hidden_dim == 8
    assert torch.equal(moe.router.expert_bias_E, torch.zeros(4))


def test_init_rng_order():
    """Router weight first, then gate/up/down interleaved per expert (moe.py:41-54)."""
    torch.manual_seed(7)
    moe = MoE(dim=6, n_experts=3, top_k=2, hidden_dim=5)
    torch.manual_seed(7)
    w_DE = torch.empty(6, 3)
    torch.nn.init.xavier_uniform_(w_DE)
    assert torch.equal(moe.router.w_DE.detach(), w_DE)
    for e in range(3):
        g, u, d = torch.empty(6, 5), torch.empty(6, 5), torch.empty(5, 6)
        for t in (g, u, d):
            torch.nn.init.xavier_uniform_(t)
        assert torch.equal(moe.w_gate_EDM[e].detach(), g)
        assert torch.equal(moe.w_up_EDM[e].detach(), u)
        assert torch.equal(moe.w_down_EMD[e].detach(), d)


def test_expert_parallel_single_process_has_identical_parameters():
    """The premise of tests/test_moe_ep.py:14-23: same seed, same parameters."""
    torch.manual_seed(0)
    a = MoE(dim=4, n_experts=4, top_k=2, hidden_dim=8, bias_update_speed=0.1)
    torch.manual_seed(0)
    b = MoEExpertParallel(dim=4, n_experts=4, top_k=2, hidden_dim=8, bias_update_speed=0.1)
    sa, sb = a.state_dict(), b.state_dict()
    assert sa.keys() == sb.keys()
    for k in sa:
        assert torch.equal(sa[k], sb[k]), k
    assert (b.rank, b.world_size) == (0, 1)


def test_constructor_errors_match_reference():
    with pytest.raises(ValueError, match=r"n_experts must be at least 1, got 0"):
        Router(4, 0, 1)
    with pytest.raises(ValueError, match=r"top_k must be in \[1, 4\], got 5"):
        Router(4, 4, 5)
    with pytest.raises(ValueError, match=r"top_k must be in \[1, 4\], got 0"):
        MoE(4, 4, 0)
    with pytest.raises(ValueError, match=r"hidden_dim must be at least 1, got 0"):
        MoE(4, 4, 2, hidden_dim=0)
    with pytest.raises(ValueError, match=r"hidden_dim must be at least 1, got -3"):
        MoEExpertParallel(4, 4, 2, hidden_dim=-3)


def test_bf16_cast_moves_bias_buffer():
    moe = MoE(8, 4, 2).to(torch.bfloat16)
    assert moe.router.expert_bias_E.dtype == torch.bfloat16
    assert moe.w_gate_EDM.dtype == torch.bfloat16


def test_other_devices_fail_loudly():
    """GPU tensors run on the HIP library and CPU tensors on its host build; any other device raises."""
    moe = MoE(8, 4, 2).to("meta")
    with pytest.raises(RuntimeError, match="ROCm"):
        moe(torch.randn(1, 3, 8, device="meta"))
    with pytest.raises(RuntimeError, match="ROCm"):
        Router(8, 4, 2).to("meta")(torch.randn(1, 3, 8, device="meta"))


def test_dense_mlp_matches_linear_layers():
    """abacus.mlp.MLP against nn.Linear (the reference's tests/test_mlp.py:6-22)."""
    torch.manual_seed(0)
    mlp = MLP(4, 8)
    x = torch.randn(2, 3, 4)
    gate, up, down = (torch.nn.Linear(4, 8, bias=False), torch.nn.Linear(4, 8, bias=False),
                      torch.nn.Linear(8, 4, bias=False))
    with torch.no_grad():
        gate.weight.copy_(mlp.w_gate_DM.T)
        up.weight.copy_(mlp.w_up_DM.T)
        down.weight.copy_(mlp.w_down_MD.T)
    torch.testing.assert_close(mlp(x), down(torch.nn.functional.silu(gate(x)) * up(x)))


# ---------------------------------------------------------------------------
# load_balancing_loss (load_balancing.py:8-41): the checks that run before any
# kernel, against the oracle's restatement of the reference
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("probs,idx", [
    (torch.tensor(1.0), torch.tensor(0)),
    (torch.zeros(3, 0), torch.zeros(3, 1, dtype=torch.long)),
    (torch.zeros(3, 4), torch.zeros(2, 1, dtype=torch.long)),
    (torch.zeros(3, 4), torch.zeros(3, 1, 1, dtype=torch.long)),
    (torch.zeros(2, 3, 4), torch.zeros(3, 2, dtype=torch.long)),
])
def test_load_balancing_value_errors_match_reference(probs, idx):
    from abacus.moe.load_balancing import load_balancing_loss
    with pytest.raises(ValueError) as want:
        oracle.load_balancing_loss(probs, idx)
    with pytest.raises(ValueError) as got:
        load_balancing_loss(probs, idx)
    assert str(got.value) == str(want.value)


def test_load_balancing_empty_and_cpu():
    from abacus.moe.load_balancing import load_balancing_loss
    z = load_balancing_loss(torch.zeros(0, 5, dtype=torch.bfloat16), torch.zeros(0, 2, dtype=torch.long))
    assert z.shape == () and z.dtype == torch.bfloat16 and float(z) == 0.0
    with pytest.raises(RuntimeError, match="ROCm"):
        load_balancing_loss(torch.rand(4, 3, device="meta"), torch.zeros(4, 1, dtype=torch.long, device="meta"))
