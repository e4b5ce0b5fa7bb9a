"""The module API on CPU tensors, through libabacus_moe_host.so (the host C++ build of the C ABI).

The reference's own CPU tests, restated: the router's known answer (tests/test_moe.py:9-39), one
expert equal to the dense MLP (tests/test_moe.py:42-53) and MoEExpertParallel in one process equal
to MoE (tests/test_moe_ep.py:14-23).  Then the layer's forward and backward against the oracle
(router.py:40-70, moe.py:60-86 restated), routing bit-exact given the library's logits, in fp32 and
bf16, with more than 64 experts and 8 slots and with D not a multiple of 8 (which the GPU kernels
reject); the
load-balancing loss; and the decoder's MoE blocks.  The host library is checked to be the code that
ran: the oracle is never on the product path.
"""

import numpy as np
import pytest
import torch

from abacus.mlp import MLP
from abacus.moe.load_balancing import load_balancing_loss
from abacus.moe.moe import MoE, MoEExpertParallel
from abacus.moe.router import Router
from abacus_amd import _lib
from abacus_amd import workloads as W
from oracle import moe_oracle as oracle
from special_selection import SPECIAL_CASES, check_special_selection


def test_router_known_answer():
    """tests/test_moe.py:9-39 on CPU tensors: expert 2 wins a slot through its bias, the bias step
    is [-10, 10, 0, 10], and the next call picks experts 3 and 1."""
    router = Router(dim=1, n_experts=4, top_k=2, bias_update_speed=10.0, route_scale=2.5)
    with torch.no_grad():
        router.w_DE.copy_(torch.tensor([[2.0, 0.0, -2.0, 1.0]]))
        router.expert_bias_E.copy_(torch.tensor([0.0, 0.0, 10.0, 0.0]))
    x = torch.ones(1, 4, 1)
    scores = torch.sigmoid(x @ router.w_DE)
    router.train()
    for bias, first in ((torch.tensor([0.0, 0.0, 10.0, 0.0]), [2]), (torch.tensor([-10.0, 10.0, 0.0, 10.0]), [3, 1])):
        weights, indices = router(x)
        want = torch.topk(scores + bias, k=2, dim=-1).indices
        picked = scores.gather(dim=-1, index=want)
        torch.testing.assert_close(indices, want)
        torch.testing.assert_close(weights, picked / picked.sum(dim=-1, keepdim=True) * router.route_scale)
        for k, e in enumerate(first):
            assert torch.all(indices[..., k] == e)
        if first == [2]:
            torch.testing.assert_close(router.expert_bias_E, torch.tensor([-10.0, 10.0, 0.0, 10.0]))


def test_one_expert_matches_mlp():
    """tests/test_moe.py:42-53 on CPU tensors."""
    torch.manual_seed(0)
    moe = MoE(4, n_experts=1, top_k=1, hidden_dim=8)
    mlp = MLP(4, 8)
    with torch.no_grad():
        mlp.w_gate_DM.copy_(moe.w_gate_EDM[0])
        mlp.w_up_DM.copy_(moe.w_up_EDM[0])
        mlp.w_down_MD.copy_(moe.w_down_EMD[0])
    x = torch.randn(2, 3, 4)
    torch.testing.assert_close(moe(x), mlp(x))


def test_one_process_expert_parallel_matches_moe():
    """tests/test_moe_ep.py:14-23 on CPU tensors: same seed, same parameters, same output and bias step."""
    torch.manual_seed(0)
    reference = MoE(dim=4, n_experts=4, top_k=2, hidden_dim=8, bias_update_speed=0.1)
    torch.manual_seed(0)
    parallel = MoEExpertParallel(dim=4, n_experts=4, top_k=2, hidden_dim=8, bias_update_speed=0.1)
    reference.train()
    parallel.train()
    x = torch.randn(2, 3, 4)
    torch.testing.assert_close(parallel(x), reference(x))
    torch.testing.assert_close(parallel.router.expert_bias_E, reference.router.expert_bias_E)


def _layer(T, D, E, K, M, dtype, seed, zipf=False):
    torch.manual_seed(seed)
    moe = MoE(D, E, K, hidden_dim=M)
    with torch.no_grad():
        for p in (moe.router.w_DE, moe.w_gate_EDM, moe.w_up_EDM, moe.w_down_EMD):
            p.normal_(0.0, 0.02 if D > 64 else 0.3)
        if zipf:
            moe.router.expert_bias_E.copy_(W.zipf_bias(E))
    x = torch.randn(T, D)
    target = torch.randn(T, D)
    return moe.to(dtype), x.to(dtype), target.to(dtype)


def _rel(got, want):
    return float((got.double() - want.double()).norm() / max(want.double().norm().item(), 1e-30))


@pytest.mark.parametrize("T,D,E,K,M,dtype", [
    (256, 128, 8, 2, 256, torch.float32),      # the tiny benchmark layer's shape
    (200, 96, 8, 3, 80, torch.bfloat16),
    (64, 20, 80, 10, 24, torch.float32),        # E > 64, K > 8, D not a multiple of 8
    (33, 64, 16, 16, 32, torch.float32),        # K == E
], ids=["tiny_f32", "bf16", "wide_E", "K_eq_E"])
def test_layer_matches_oracle(T, D, E, K, M, dtype):
    moe, x, target = _layer(T, D, E, K, M, dtype, seed=T + E)
    moe.train()
    bias0 = moe.router.expert_bias_E.detach().clone()
    xr = x.clone().requires_grad_()
    out = moe(xr)
    ((out.float() - target.float()) ** 2).mean().backward()
    r = moe.router.last_routing

    # routing: bit-exact against the oracle given the library's logits; counts, offsets, permutation
    w_o, idx_o, _ = oracle.route(r.logits_TE, bias0, K, moe.router.route_scale)
    assert torch.equal(r.indices_TK, idx_o)
    assert torch.equal(r.weights_TK, w_o)
    counts, offsets, perm, pos = oracle.dispatch(idx_o, E)
    assert np.array_equal(r.counts_E.numpy(), counts) and np.array_equal(r.offsets_E1.numpy(), offsets)
    assert np.array_equal(r.perm_R.numpy(), perm) and np.array_equal(r.pos_TK.numpy(), pos)
    assert torch.equal(moe.router.expert_bias_E, oracle.bias_step(bias0, idx_o, E, moe.router.bias_update_speed))

    # outputs and gradients: against the oracle in fp64 on the same routing
    names = ("router.w_DE", "w_gate_EDM", "w_up_EDM", "w_down_EMD")
    params = {n: p.detach().double().requires_grad_() for n, p in moe.named_parameters()}
    x64 = x.double().requires_grad_()
    ref, _ = oracle.moe_forward(x64, *(params[n] if n == "router.w_DE" else None for n in names[:1]),
                                bias0.double(), params["w_gate_EDM"], params["w_up_EDM"], params["w_down_EMD"], K,
                                indices_TK=idx_o)
    ((ref - target.double()) ** 2).mean().backward()
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert _rel(out.detach(), ref.detach()) < tol
    assert _rel(xr.grad, x64.grad) < tol
    for n, p in moe.named_parameters():
        assert _rel(p.grad, params[n].grad) < tol, n


def test_cpu_calls_run_the_host_library(monkeypatch):
    """Every library call of a CPU forward + backward goes to libabacus_moe_host.so; the oracle is
    not imported by the product path and the HIP library is not called."""
    called = []
    real = _lib.load_host

    def spy():
        lib = real()

        class Spy:
            def __getattr__(self, name):
                called.append(name)
                return getattr(lib, name)
        return Spy()

    monkeypatch.setattr(_lib, "load_host", spy)
    monkeypatch.setattr(_lib, "load", lambda: (_ for _ in ()).throw(AssertionError("HIP library called")))
    moe, x, target = _layer(40, 16, 4, 2, 24, torch.float32, seed=3)
    xr = x.requires_grad_()
    ((moe(xr) - target) ** 2).mean().backward()
    for name in ("abacus_moe_router_fwd", "abacus_moe_dispatch",
                 "abacus_moe_gateup_fwd", "abacus_moe_down_fwd", "abacus_moe_combine_fwd", "abacus_moe_combine_bwd",
                 "abacus_moe_down_bwd", "abacus_moe_gateup_bwd", "abacus_moe_unpermute_bwd", "abacus_moe_router_wgrad"):
        assert name in called, name
    import abacus_amd.moe as product
    assert "oracle" not in product.__dict__


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_router_alone_backward_matches_fp64(dtype):
    torch.manual_seed(11)
    T, D, E, K = 50, 64, 8, 3
    router = Router(D, E, K, route_scale=1.5).to(dtype)
    x = torch.randn(T, D, dtype=dtype, requires_grad=True)
    g = torch.randn(T, K, dtype=dtype)
    router.eval()
    w, idx = router(x)
    (w.float() * g.float()).sum().backward()
    x_ref = x.detach().double().requires_grad_()
    wde = router.w_DE.detach().double().requires_grad_()
    picked = torch.sigmoid(x_ref @ wde).gather(-1, idx)
    ((picked / picked.sum(-1, keepdim=True) * 1.5) * g.double()).sum().backward()
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert _rel(x.grad, x_ref.grad) < tol and _rel(router.w_DE.grad, wde.grad) < tol


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_load_balancing_matches_oracle(dtype):
    torch.manual_seed(5)
    probs = torch.rand(3, 70, 12).to(dtype).requires_grad_()
    idx = torch.randint(0, 12, (3, 70, 4))
    loss = load_balancing_loss(probs, idx)
    loss.backward()
    p2 = probs.detach().clone().requires_grad_()
    want = oracle.load_balancing_loss(p2, idx)
    want.backward()
    tol = 1e-5 if dtype == torch.float32 else 8e-3
    assert abs(float(loss) - float(want)) <= tol * abs(float(want))
    assert _rel(probs.grad, p2.grad) < (1e-6 if dtype == torch.float32 else 8e-3)
    with pytest.raises(RuntimeError, match="non-negative"):
        load_balancing_loss(torch.rand(4, 3), torch.tensor([[0], [-1], [1], [2]]))


def test_decoder_moe_blocks_train_on_cpu():
    """TransformerMoe (transformer_moe.py:17-75) on CPU tensors: its MoE layers run on the host
    library; one training step gives a finite loss and moves every router's bias."""
    from abacus.transformer_moe import TransformerMoe
    from abacus_amd.train import make_optimizer, train_step
    torch.manual_seed(4)
    model = TransformerMoe(dim=32, n_heads=2, head_dim=16, n_blocks=2, vocab_size=101, n_experts=4, top_k=2,
                           hidden_dim=48)
    tokens = torch.randint(0, 101, (2, 24))
    bias0 = [b.moe.router.expert_bias_E.clone() for b in model.blocks]
    loss = train_step(model, make_optimizer(model), tokens)
    assert torch.isfinite(loss)
    assert all(not torch.equal(b0, b.moe.router.expert_bias_E) for b0, b in zip(bias0, model.blocks))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_adamw_on_cpu_matches_oracle(dtype):
    """AdamW's CPU step (the reference's torch ops, optimizers/adamw.py:107-119) against the oracle's
    restatement over three steps: within one bf16 ulp, or 1e-6 relative in fp32 (torch's CPU lerp,
    addcmul and addcdiv round differently from the GPU forms the oracle follows; measured: bf16
    identical, fp32 at most 4.2e-7 on 1.3% of the elements)."""
    from abacus_amd.optim import AdamW
    from oracle.adamw_oracle import adamw_step
    hp = dict(lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=1e-2)
    g = torch.Generator().manual_seed(7)
    model = torch.nn.ParameterList([torch.nn.Parameter((torch.randn(n, generator=g) * 0.5).to(dtype))
                                    for n in (1, 7, 1000)])
    opt = AdamW(model, lr=hp["lr"], betas=(hp["beta1"], hp["beta2"]), eps=hp["eps"], weight_decay=hp["weight_decay"])
    ora = [[p.detach().float().numpy(), np.zeros(p.numel(), np.float32), np.zeros(p.numel(), np.float32)]
           for p in model]
    name = "bf16" if dtype == torch.bfloat16 else "fp32"
    for step in range(1, 4):
        for i, p in enumerate(model):
            p.grad = (torch.randn(p.shape, generator=g) * 10.0 ** (step - 2)).to(dtype)
            ora[i] = list(adamw_step(*ora[i][:1], p.grad.float().numpy(), ora[i][1], ora[i][2], step, dtype=name, **hp))
        opt.step()
    ulp = 2.0 ** -7 if dtype == torch.bfloat16 else 1e-6
    for p, o in zip(model, ora):
        got, want = p.detach().double().numpy(), o[0].astype(np.float64)
        assert np.all(np.abs(got - want) <= ulp * np.abs(want) + 1e-30)


@pytest.mark.parametrize("E,K,dtype", SPECIAL_CASES, ids=[f"E{e}_K{k}_{str(d)[6:]}" for e, k, d in SPECIAL_CASES])
def test_selection_order_special_values_on_cpu(E, K, dtype):
    """NaN, +-inf, exact ties and zero selections on the host build: see tests/special_selection.py."""
    check_special_selection(E, K, dtype, torch.device("cpu"))
