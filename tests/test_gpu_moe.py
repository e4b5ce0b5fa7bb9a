"""MoE layer forward + backward on the GPU against the oracle: on the CPU at sizes it finishes
in seconds, and as the same torch ops on the GPU at the full workload sizes.  Routing is taken
from the kernel (identical-logits contract) so both sides run the same experts.

Tolerances (the layer's contract: rtol 1e-5 in fp32, 2e-2 in bf16) are applied against an
fp64 evaluation of the same algorithm, allowing exactly the error the reference's own
computation in the workload dtype incurs; see check_against.
"""

import pytest
import torch

from abacus_amd import _lib
from abacus_amd import workloads as W
from abacus.mlp import MLP
from abacus.moe.moe import MoE, MoEExpertParallel
from bench_inputs import bench_inputs
from oracle import moe_oracle as oracle

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)
PARAMS = ("router.w_DE", "w_gate_EDM", "w_up_EDM", "w_down_EMD")


def rtol_for(dtype):
    return 1e-5 if dtype == torch.float32 else 2e-2


def rms(t):
    return float(t.float().pow(2).mean().sqrt()) if t.numel() else 0.0


def assert_close_scaled(got, want, rtol, what):
    got, want = got.float().cpu(), want.float().cpu()
    atol = rtol * max(rms(want), 1e-30)
    torch.testing.assert_close(got, want, rtol=rtol, atol=atol, msg=lambda m: f"{what}: {m}")


def rel_err(got, want):
    """Normwise relative error ||got - want|| / ||want||."""
    got, want = got.double().cpu(), want.double().cpu()
    return float((got - want).norm() / max(float(want.norm()), 1e-300))


def product_step(moe, x, target, backward=True):
    """One forward (+ MSE backward) through the HIP path; returns out, x.grad, param grads, routing."""
    x = x.detach().clone().requires_grad_(backward)
    moe.zero_grad(set_to_none=True)
    out = moe(x)
    grads = {}
    if backward:
        loss = (out.float() - target.float()).pow(2).mean()
        loss.backward()
        grads = {n: p.grad for n, p in moe.named_parameters()}
    torch.cuda.synchronize()
    return out.detach(), (x.grad if backward else None), grads, moe.router.last_routing


def reference_step(moe, x, target, indices, compute_dtype, device, backward=True):
    """The oracle (reference algorithm) with the given routing, in compute_dtype on device."""
    p = {n: t.detach().to(device=device, dtype=compute_dtype).clone().requires_grad_(backward)
         for n, t in moe.named_parameters()}
    bias = moe.router.expert_bias_E.detach().to(device=device, dtype=compute_dtype)
    xr = x.detach().to(device=device, dtype=compute_dtype).clone().requires_grad_(backward)
    x_TD = xr.reshape(-1, moe.dim)
    out, _ = oracle.moe_forward(x_TD, p["router.w_DE"], bias, p["w_gate_EDM"], p["w_up_EDM"], p["w_down_EMD"],
                                moe.top_k, moe.router.route_scale, indices_TK=indices.to(device))
    out = out.reshape(x.shape)
    grads = {}
    if backward:
        loss = (out.double() - target.to(device).double()).pow(2).mean()
        loss.backward()
        grads = {n: t.grad for n, t in p.items()}
    return out.detach(), (xr.grad if backward else None), grads


def _named(out, dx, grads, backward):
    t = {"out": out}
    if backward:
        t["dx"] = dx
        for n in PARAMS:
            t["d" + n] = grads[n]
    return t


def check_against(moe, x, target, device, backward=True):
    """Kernel vs the reference algorithm, judged against an fp64 evaluation ("truth").

    For every output and gradient, with rtol = 1e-5 (fp32) or 2e-2 (bf16):
      normwise     ||kernel - truth|| / ||truth|| <= max(rtol, 1.25 * that of the reference
                   evaluated in the workload dtype with the reference's op-by-op rounding)
      elementwise  max |kernel - truth| <= 2 * max |reference - truth| + rtol * rms(truth)
    i.e. within the contract tolerance of the exact result, or no less accurate than the
    reference's own computation in that dtype (two evaluations in one dtype differ from each
    other on near-cancelling entries by more than rtol * rms, so the dtype reference cannot
    referee elementwise on its own).
    K == 1: the router gradients are exactly zero (w = rho * s / s); the kernel must return
    zeros and the comparison skips them.
    """
    moe.eval()  # no bias drift between the evaluations
    dtype = moe.w_gate_EDM.dtype
    out, dx, grads, routing = product_step(moe, x, target, backward)
    idx = routing.indices_TK.reshape(-1, moe.top_k)
    got = _named(out, dx, grads, backward)
    truth = _named(*reference_step(moe, x, target, idx, torch.float64, device, backward), backward)
    ref = _named(*reference_step(moe, x, target, idx, dtype, device, backward), backward)
    rtol = rtol_for(dtype)
    for name in got:
        if moe.top_k == 1 and name == "drouter.w_DE":
            assert torch.count_nonzero(got[name]) == 0
            continue
        t = truth[name].double().cpu()
        k = got[name].double().cpu()
        r = ref[name].double().cpu()
        e_k, e_r = rel_err(k, t), rel_err(r, t)
        m_k, m_r = float((k - t).abs().max()), float((r - t).abs().max())
        scale = rms(t)
        print(f"  {name:16s} normwise kernel {e_k:.2e} ref({str(dtype)[6:]}) {e_r:.2e}   "
              f"max/rms kernel {m_k / max(scale, 1e-300):.2e} ref {m_r / max(scale, 1e-300):.2e}", flush=True)
        assert e_k <= max(rtol, 1.25 * e_r), f"{name}: normwise error {e_k:.3e}"
        assert m_k <= 2 * m_r + rtol * scale, f"{name}: max error {m_k:.3e} vs reference {m_r:.3e}"


# ---------------- oracle on the CPU, same dtype ----------------
ORACLE_CASES = [
    (W.TINY_F32, True),
    (W.MID_F32.with_tokens(1, 1024), True),
    (W.SKEW_BF16_T64, False),
]


@pytest.mark.parametrize("wl,backward", ORACLE_CASES, ids=[c[0].name for c in ORACLE_CASES])
def test_matches_cpu_oracle(wl, backward):
    print(f"\n[moe-oracle] {wl.name} dtype={wl.dtype} bwd={backward}", flush=True)
    small = wl.dim * wl.hidden * wl.n_experts < 50_000_000
    moe, x, target = W.build(wl, device=DEV) if small else W.build_on_device(wl, DEV)
    check_against(moe, x, target, torch.device("cpu"), backward)


# ---------------- the oracle's torch ops on the GPU, full sizes ----------------
# On the exact inputs bench.py times (the host recipe), and on a second draw of every workload's
# distributions made on the GPU.
FULL_CASES = [W.TINY_F32, W.MID_F32, W.MIXTRAL_BF16, W.SKEW_BF16_T64, W.SKEW_BF16_T512, W.SKEW_BF16_T16K,
              W.FINE_BF16]


@pytest.mark.parametrize("wl", FULL_CASES, ids=[w.name for w in FULL_CASES])
def test_matches_reference_full_size(wl):
    print(f"\n[moe-full] {wl.name} T={wl.tokens} D={wl.dim} E={wl.n_experts} K={wl.top_k} M={wl.hidden} "
          f"bwd={wl.backward} (bench inputs)", flush=True)
    moe, x, target = bench_inputs(wl, DEV)
    check_against(moe, x, target, DEV, wl.backward)


@pytest.mark.parametrize("wl", FULL_CASES, ids=[w.name for w in FULL_CASES])
def test_matches_reference_full_size_device_draw(wl):
    print(f"\n[moe-full] {wl.name} (values drawn on the GPU)", flush=True)
    moe, x, target = W.build_on_device(wl, DEV)
    check_against(moe, x, target, DEV, wl.backward)


# ---------------- edge cases (the reference's own test scenarios) ----------------
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_one_expert_matches_mlp(dtype):
    """tests/test_moe.py:42-53 on the GPU (E = 1, K = 1 is the dense SwiGLU)."""
    torch.manual_seed(0)
    moe = MoE(4 if dtype == torch.float32 else 8, n_experts=1, top_k=1, hidden_dim=8)
    mlp = MLP(moe.dim, 8)
    with torch.no_grad():
        mlp.w_gate_DM.copy_(moe.w_gate_EDM[0])
        mlp.w_up_DM.copy_(moe.w_up_EDM[0])
        mlp.w_down_MD.copy_(moe.w_down_EMD[0])
    moe, mlp = moe.to(DEV, dtype), mlp.to(DEV, dtype)
    x = torch.randn(2, 3, moe.dim, device=DEV, dtype=dtype)
    rtol = rtol_for(dtype)
    assert_close_scaled(moe(x), mlp(x), rtol, "out")


def test_forced_routing_leaves_experts_empty():
    """w_DE = -8 except column 0 = +8, speed 0 (tests/test_moe_ep.py:94-102): experts 1..3 empty."""
    torch.manual_seed(2)
    moe = MoE(dim=4, n_experts=4, top_k=1, hidden_dim=8, bias_update_speed=0.0)
    with torch.no_grad():
        moe.router.w_DE.fill_(-8)
        moe.router.w_DE[:, 0] = 8
    moe = moe.to(DEV)
    # positive inputs: logit(expert 0) = 8 sum(x) > 0 > -8 sum(x) for every other expert
    x = torch.randn(2, 3, 4, device=DEV).abs() + 0.1
    target = torch.randn(2, 3, 4, device=DEV)
    moe.train()
    out, dx, grads, routing = product_step(moe, x, target)
    assert routing.counts_E.tolist() == [6, 0, 0, 0]
    assert routing.offsets_E1.tolist() == [0, 6, 6, 6, 6]
    for n in ("w_gate_EDM", "w_up_EDM", "w_down_EMD"):
        assert torch.count_nonzero(grads[n][1:]) == 0
    check_against(moe, x, target, torch.device("cpu"))


def test_tied_logits_follow_lower_index_rule():
    """With x of mixed sign the reference's forced-routing inputs tie experts 1..3 (tests/test_moe_ep.py:94-102):
    the kernel resolves the tie to the lowest index, like the oracle."""
    torch.manual_seed(2)
    moe = MoE(dim=4, n_experts=4, top_k=1, hidden_dim=8, bias_update_speed=0.0)
    with torch.no_grad():
        moe.router.w_DE.fill_(-8)
        moe.router.w_DE[:, 0] = 8
    moe = moe.to(DEV)
    x = torch.randn(2, 3, 4, device=DEV)
    moe.eval()
    with torch.no_grad():
        moe(x)
    r = moe.router.last_routing
    positive = (x.reshape(-1, 4).sum(-1) > 0).cpu()
    assert r.indices_TK.reshape(-1).cpu().tolist() == [0 if p else 1 for p in positive.tolist()]


@pytest.mark.parametrize("T,E,K,rs", [(1, 4, 1, 1.0), (6, 4, 2, 1.5), (37, 8, 3, 1.0), (100, 16, 8, 0.7)])
def test_small_ragged_shapes(T, E, K, rs):
    """Token counts off the 16-token block, K up to 8, single-token batches (three empty experts)."""
    print(f"\n[moe-small] T={T} E={E} K={K} rs={rs}", flush=True)
    torch.manual_seed(T + E)
    moe = MoE(dim=16, n_experts=E, top_k=K, hidden_dim=24, route_scale=rs).to(DEV)
    x = torch.randn(1, T, 16, device=DEV)
    target = torch.randn(1, T, 16, device=DEV)
    check_against(moe, x, target, torch.device("cpu"))


@pytest.mark.parametrize("T,D,M,E,K", [(50, 72, 200, 5, 2), (130, 136, 264, 12, 3), (300, 192, 320, 3, 1),
                                        (7, 64, 64, 64, 8), (600, 128, 128, 6, 2),
                                        (512, 128, 128, 8, 2), (513, 128, 128, 8, 2)])  # R = 128 E: thin / full
def test_bf16_odd_shapes(T, D, M, E, K):
    """bf16 layers at sizes the workloads do not reach: D and M multiples of 8 but not of 64
    (the generic kernel), E = 64 with K = 8 and nearly every expert empty or tiny (thin tiles,
    the down projection's small-batch path), experts holding full tiles plus a remainder;
    forward and backward against the oracle."""
    print(f"\n[moe-bf16-odd] T={T} D={D} M={M} E={E} K={K}", flush=True)
    torch.manual_seed(T * 7 + D)
    moe = MoE(dim=D, n_experts=E, top_k=K, hidden_dim=M).to(torch.bfloat16).to(DEV)
    x = torch.randn(1, T, D, device=DEV).to(torch.bfloat16)
    target = torch.randn(1, T, D, device=DEV).to(torch.bfloat16)
    check_against(moe, x, target, torch.device("cpu"))


@pytest.mark.parametrize("T,D,M,E,K,dtype", [
    (300, 256, 128, 128, 8, torch.bfloat16),
    (200, 128, 64, 256, 16, torch.float32),
    (500, 512, 256, 80, 10, torch.bfloat16),
    (257, 64, 96, 65, 1, torch.float32),
    (300, 128, 64, 300, 20, torch.bfloat16),
    (200, 64, 32, 1024, 64, torch.float32),
    (256, 128, 64, 40, 24, torch.bfloat16),
    (300, 72, 64, 513, 8, torch.bfloat16),
    (8192, 128, 64, 256, 8, torch.bfloat16),
    (8200, 64, 32, 384, 8, torch.bfloat16),
], ids=["E128_K8_bf16", "E256_K16_f32", "E80_K10_bf16", "E65_K1_f32", "E300_K20_bf16", "E1024_K64_f32",
        "E40_K24_bf16", "E513_K8_bf16", "E256_K8_T8192_bf16", "E384_K8_T8200_bf16"])
def test_wide_expert_counts(T, D, M, E, K, dtype):
    """Router sizes beyond 64 experts and 8 slots, up to the library's 1024 and 64 (past 256
    experts or 16 slots the router runs as a logits pass and a top-k pass, and the dispatch and
    backward kernels take their 64-slot forms; the reference's Router takes any E >= 1,
    1 <= K <= E, router.py:25-28): routing bit-exact against the oracle on the kernel's logits,
    then the layer against the oracle."""
    print(f"\n[moe-wide] T={T} D={D} M={M} E={E} K={K} {dtype}", flush=True)
    torch.manual_seed(E + K)
    moe = MoE(D, E, K, hidden_dim=M)
    with torch.no_grad():
        for p in (moe.router.w_DE, moe.w_gate_EDM, moe.w_up_EDM, moe.w_down_EMD):
            p.normal_(0.0, 0.05)
    moe = moe.to(DEV, dtype)
    x = torch.randn(T, D, device=DEV).to(dtype)
    target = torch.randn(T, D, device=DEV).to(dtype)
    moe.train()
    bias0 = moe.router.expert_bias_E.detach().clone()
    with torch.no_grad():
        moe(x)
    torch.cuda.synchronize()
    r = moe.router.last_routing
    w_o, idx_o, _ = oracle.route(r.logits_TE.cpu(), bias0.cpu(), K, moe.router.route_scale)
    assert torch.equal(r.indices_TK.cpu(), idx_o)
    assert torch.equal(r.weights_TK.cpu(), w_o)
    counts, offsets, perm, pos = oracle.dispatch(idx_o, E)
    assert r.counts_E.cpu().tolist() == counts.tolist() and r.offsets_E1.cpu().tolist() == offsets.tolist()
    assert r.perm_R.cpu().tolist() == perm.tolist() and r.pos_TK.cpu().reshape(-1).tolist() == pos.reshape(-1).tolist()
    assert torch.equal(moe.router.expert_bias_E.cpu(), oracle.bias_step(bias0.cpu(), idx_o, E, moe.router.bias_update_speed))
    check_against(moe, x, target, torch.device("cpu"))


@pytest.mark.parametrize("T,D,M,E,K,dtype", [
    (37, 20, 36, 5, 2, torch.bfloat16),
    (64, 6, 10, 4, 2, torch.float32),
    (50, 4, 4, 3, 1, torch.bfloat16),
    (300, 130, 200, 8, 2, torch.bfloat16),
], ids=["D20_M36_bf16", "D6_M10_f32", "D4_M4_bf16", "D130_M200_bf16"])
def test_dims_off_the_vector_width(T, D, M, E, K, dtype):
    """D or M not a multiple of the kernels' 16-byte vectors (8 bf16, 4 fp32): the layer zero-pads
    them for the GPU kernels, as the reference takes any dim (moe.py:25-57); forward and backward
    against the oracle, routing bit-exact on the kernel's logits, gradients in the parameters'
    shapes."""
    print(f"\n[moe-pad] T={T} D={D} M={M} E={E} K={K} {dtype}", flush=True)
    torch.manual_seed(T + D + M)
    moe = MoE(dim=D, n_experts=E, top_k=K, hidden_dim=M).to(dtype).to(DEV)
    x = torch.randn(1, T, D, device=DEV).to(dtype)
    target = torch.randn(1, T, D, device=DEV).to(dtype)
    moe.train()
    bias0 = moe.router.expert_bias_E.detach().clone()
    xr = x.clone().requires_grad_()
    out = moe(xr)
    ((out.float() - target.float()) ** 2).mean().backward()
    assert out.shape == x.shape and xr.grad.shape == x.shape
    for n, p in moe.named_parameters():
        assert p.grad is not None and p.grad.shape == p.shape, n
    r = moe.router.last_routing
    w_o, idx_o, _ = oracle.route(r.logits_TE.cpu(), bias0.cpu(), K, moe.router.route_scale)
    assert torch.equal(r.indices_TK.cpu(), idx_o) and torch.equal(r.weights_TK.cpu(), w_o)
    moe.router.expert_bias_E.copy_(bias0)
    check_against(moe, x, target, torch.device("cpu"))


def test_two_training_steps_track_bias_updates():
    """Two train-mode iterations (tests/test_moe_ep.py:49-71): outputs, grads and the bias."""
    torch.manual_seed(1)
    moe = MoE(dim=16, n_experts=4, top_k=2, hidden_dim=32, bias_update_speed=0.25, route_scale=1.5).to(DEV)
    moe.train()
    bias = moe.router.expert_bias_E.detach().cpu().clone()
    for step in range(2):
        x = torch.randn(2, 9, 16, device=DEV)
        target = torch.randn(2, 9, 16, device=DEV)
        out, dx, grads, routing = product_step(moe, x, target)
        logits = routing.logits_TE.cpu()
        _, idx_o, _ = oracle.route(logits, bias, 2, 1.5)
        assert torch.equal(routing.indices_TK.cpu(), idx_o), step
        bias = oracle.bias_step(bias, idx_o, 4, 0.25)
        assert torch.equal(moe.router.expert_bias_E.cpu(), bias), step
        # the oracle (fp64) reproduces the output and input gradient with the same routing
        r_out, r_dx, _ = reference_step(moe, x, target, idx_o, torch.float64, torch.device("cpu"))
        assert_close_scaled(out, r_out, 1e-5, "out")
        assert_close_scaled(dx, r_dx, 1e-5, "dx")


def test_one_process_expert_parallel_matches_moe():
    """tests/test_moe_ep.py:14-23 on the GPU: MoEExpertParallel at world size 1 == MoE."""
    torch.manual_seed(0)
    ref = MoE(dim=4, n_experts=4, top_k=2, hidden_dim=8, bias_update_speed=0.1).to(DEV)
    torch.manual_seed(0)
    par = MoEExpertParallel(dim=4, n_experts=4, top_k=2, hidden_dim=8, bias_update_speed=0.1).to(DEV)
    ref.train()
    par.train()
    x = torch.randn(2, 3, 4, device=DEV)
    torch.testing.assert_close(par(x), ref(x))
    torch.testing.assert_close(par.router.expert_bias_E, ref.router.expert_bias_E)


@pytest.mark.parametrize("wl", [W.TINY_F32, W.SKEW_BF16_T512.with_tokens(1, 1000)], ids=["tiny_f32", "skew_bf16_T1000"])
def test_deterministic(wl):
    """No atomics on the data path: two runs are bitwise identical."""
    moe, x, target = W.build_on_device(dataclasses_replace_backward(wl), DEV)
    moe.eval()
    a = product_step(moe, x, target)
    b = product_step(moe, x, target)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])
    for n in PARAMS:
        assert torch.equal(a[2][n], b[2][n]), n


def dataclasses_replace_backward(wl):
    import dataclasses
    return dataclasses.replace(wl, backward=True)


def test_empty_batch_returns_input():
    moe = MoE(8, 4, 2).to(DEV)
    x = torch.randn(2, 0, 8, device=DEV)
    assert moe(x) is x


def test_native_library_is_what_ran():
    moe = MoE(8, 4, 2).to(DEV)
    moe(torch.randn(1, 5, 8, device=DEV))
    assert _lib._lib is not None and str(_lib.LIB_PATH).endswith("libabacus_moe.so")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("rs", [1.5, 0.75, 2.5])
def test_one_slot_router_gradient_is_exactly_zero(dtype, rs):
    """With top_k = 1 the weight is route_scale * s / s = route_scale, so the router's gradients are exactly
    zero (router.py:49-51).  The gating backward's products are rounded on their own: an fma of
    route_scale * dw - dw * w had left one product's rounding error in every dlogit (about 1e-9 in dW_DE)
    when route_scale * dw is not exact."""
    torch.manual_seed(3)
    moe = MoE(256, 4, 1, hidden_dim=16, route_scale=rs)
    with torch.no_grad():
        for p in (moe.router.w_DE, moe.w_gate_EDM, moe.w_up_EDM, moe.w_down_EMD):
            p.normal_(0.0, 0.1)
    moe = moe.to(DEV, dtype)
    moe.eval()
    x = torch.randn(300, 256, device=DEV).to(dtype).requires_grad_()
    out = moe(x)
    ((out.float() - 1.0) ** 2).mean().backward()
    torch.cuda.synchronize()
    assert torch.count_nonzero(moe.router.w_DE.grad) == 0
    assert torch.isfinite(x.grad).all()
