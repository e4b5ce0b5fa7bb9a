"""Routing parity on the GPU: indices, weights, per-expert counts, offsets, the permutation
and the bias step are bit-exact against the oracle given the kernel's own logits
(router.py:40-70, moe.py:72-77); against torch.sigmoid + torch.topk they pick the same set
on every token without a boundary tie or a boundary sigmoid difference, and a valid top-k
under torch's values on those (tests/routing_check.py)."""

import numpy as np
import pytest
import torch

from abacus_amd import workloads as W
from abacus.moe.router import Router
from bench_inputs import bench_inputs
from oracle import moe_oracle as oracle
from routing_check import check_against_torch_topk
from special_selection import LARGE_BATCH_CASES, SPECIAL_CASES, check_special_selection

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)

# (workload, the exact inputs bench.py times?)  Otherwise a second draw of the same
# distributions, made on the GPU.
WORKLOADS = [W.TINY_F32, W.MID_F32, W.MIXTRAL_BF16, W.SKEW_BF16_T64, W.SKEW_BF16_T512, W.SKEW_BF16_T16K,
             W.FINE_BF16]
CASES = [(w, True) for w in WORKLOADS] + [(w, False) for w in WORKLOADS if w.dim * w.n_experts >= 2**16]


def build(wl, bench):
    if bench:
        return bench_inputs(wl, DEV)
    return W.build_on_device(wl, DEV)


@pytest.mark.parametrize("wl,bench", CASES, ids=[c[0].name + ("" if c[1] else "-device_draw") for c in CASES])
def test_routing_bit_exact(wl, bench):
    print(f"\n[routing] {wl.name} T={wl.tokens} D={wl.dim} E={wl.n_experts} K={wl.top_k} "
          f"{'bench inputs' if bench else 'drawn on the GPU'}", flush=True)
    moe, x, _ = build(wl, bench)
    moe.train()
    bias0 = moe.router.expert_bias_E.detach().clone()
    with torch.no_grad():
        moe(x)
    torch.cuda.synchronize()
    r = moe.router.last_routing
    E, K = wl.n_experts, wl.top_k
    logits = r.logits_TE.cpu()
    w_o, idx_o, _ = oracle.route(logits, bias0.cpu(), K, moe.router.route_scale)
    idx_k = r.indices_TK.cpu()
    assert torch.equal(idx_k, idx_o)
    assert torch.equal(r.weights_TK.cpu(), w_o)
    counts, offsets, perm, pos = oracle.dispatch(idx_o, E)
    assert np.array_equal(r.counts_E.cpu().numpy(), counts)
    assert np.array_equal(r.offsets_E1.cpu().numpy(), offsets)
    assert np.array_equal(r.perm_R.cpu().numpy(), perm)
    assert np.array_equal(r.pos_TK.cpu().numpy(), pos)
    bias_o = oracle.bias_step(bias0.cpu(), idx_o, E, moe.router.bias_update_speed)
    assert torch.equal(moe.router.expert_bias_E.cpu(), bias_o)

    # The logits themselves are a GEMM: close to an fp32 product of the same inputs.
    ref = x.float().reshape(-1, wl.dim) @ moe.router.w_DE.float()
    tol = 1e-5 if wl.dtype == torch.float32 else 1e-2
    torch.testing.assert_close(r.logits_TE.float(), ref, rtol=tol, atol=tol * float(ref.std()))

    # Against the literal reference ops: the same set wherever torch's values leave no choice.
    _, _, scores_cr = oracle.route(logits, bias0.cpu(), K, moe.router.route_scale)
    c = check_against_torch_topk(logits, bias0.cpu(), idx_k, scores_cr)
    print(f"[routing] {wl.name} vs torch.sigmoid+torch.topk: {c.summary()}", flush=True)
    assert c.set_mismatches == 0 and c.invalid_exempt == 0
    assert c.sigmoid_exempt <= max(2, c.tokens // 100)
    if wl.dtype == torch.float32:
        assert c.exempt == 0


def test_router_known_answer():
    """The reference's router test (tests/test_moe.py:9-39) through the kernel, dim = 1."""
    router = Router(dim=1, n_experts=4, top_k=2, bias_update_speed=10.0, route_scale=2.5).to(DEV)
    with torch.no_grad():
        router.w_DE.copy_(torch.tensor([[2.0, 0.0, -2.0, 1.0]]))
        router.expert_bias_E.copy_(torch.tensor([0.0, 0.0, 10.0, 0.0]))
    x = torch.ones(1, 4, 1, device=DEV)
    scores = torch.sigmoid(x @ router.w_DE)
    router.train()
    weights, indices = router(x)
    start = torch.tensor([0.0, 0.0, 10.0, 0.0], device=DEV)
    expected = torch.topk(scores + start, k=2, dim=-1).indices
    picked = scores.gather(dim=-1, index=expected)
    torch.testing.assert_close(indices, expected)
    torch.testing.assert_close(weights, picked / picked.sum(dim=-1, keepdim=True) * 2.5)
    assert torch.all(indices[..., 0] == 2)
    assert router.expert_bias_E.tolist() == [-10.0, 10.0, 0.0, 10.0]
    weights2, indices2 = router(x)
    stepped = torch.tensor([-10.0, 10.0, 0.0, 10.0], device=DEV)
    expected2 = torch.topk(scores + stepped, k=2, dim=-1).indices
    picked2 = scores.gather(dim=-1, index=expected2)
    torch.testing.assert_close(indices2, expected2)
    torch.testing.assert_close(weights2, picked2 / picked2.sum(dim=-1, keepdim=True) * 2.5)
    assert torch.all(indices2[..., 0] == 3) and torch.all(indices2[..., 1] == 1)


@pytest.mark.parametrize("E,K", [(8, 3), (300, 20), (64, 40)], ids=["E8_K3", "E300_K20", "E64_K40"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_router_backward_matches_oracle(dtype, E, K):
    """Standalone Router: gradients of sum(weights * g) w.r.t. x and w_DE (past 256 experts or 16
    slots: the wide router, the slot-loop gating backward and the 64-slot weight gradient)."""
    torch.manual_seed(11 + E + K)
    T, D = 50, 64
    router = Router(D, E, K, route_scale=1.5).to(device=DEV, dtype=dtype)
    x = torch.randn(T, D, device=DEV, dtype=dtype, requires_grad=True)
    g = torch.randn(T, K, device=DEV, dtype=dtype)
    router.eval()
    w, idx = router(x)
    (w.float() * g.float()).sum().backward()
    x_ref = x.detach().cpu().double().requires_grad_()
    wde_ref = router.w_DE.detach().cpu().double().requires_grad_()
    logits = x_ref @ wde_ref
    s = torch.sigmoid(logits)
    picked = s.gather(-1, idx.cpu())
    w_ref = picked / picked.sum(-1, keepdim=True) * 1.5
    (w_ref * g.cpu().double()).sum().backward()
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    for got, want in ((x.grad, x_ref.grad), (router.w_DE.grad, wde_ref.grad)):
        want = want.float()
        torch.testing.assert_close(got.float().cpu(), want, rtol=tol, atol=tol * float(want.pow(2).mean().sqrt()))


@pytest.mark.parametrize("T,D,E,K", [(1, 64, 8, 2), (16, 4096, 32, 2), (700, 2048, 48, 4), (1024, 264, 64, 6),
                                     (1025, 264, 64, 6), (300, 520, 128, 8), (64, 1032, 256, 8), (33, 2048, 160, 6),
                                     (1024, 1024, 256, 16), (8200, 264, 256, 8), (8192, 136, 160, 16),
                                     (8250, 72, 512, 8), (8210, 128, 264, 4)])
def test_router_small_batch_slices(T, D, E, K):
    """bf16 routers with at most 256 experts and at most 1024 tokens sum the logits over 8 slices of D
    in a second launch (at D = 264 the last three slices are empty; 1025 tokens take the one-launch
    path; 160 experts pad to 256).  From 8192 tokens with 129 or more experts the router runs
    64-token blocks sharing staged weight rows (with 512 and 264 experts as the logits pass over
    groups of 256 before the top-k pass; T = 8200, 8210, 8250 leave partial 64-token and 16-token
    blocks).  Through the C ABI: the transposed weight the slice blocks write into the workspace is
    exactly w_DE^T (zero rows past E) and the block histograms count the picks.  Through the module:
    routing bit-exact against the oracle given the kernel's logits, logits close to an fp32
    product, input and weight gradients close to fp64 (xavier-initialised weights, logits O(1))."""
    from abacus_amd._lib import call, ptr, query, stream_of, dtype_code
    print(f"\n[router-slices] T={T} D={D} E={E} K={K}", flush=True)
    gen = torch.Generator().manual_seed(T * 7 + D)
    router = Router(D, E, K, route_scale=1.5).to(device=DEV, dtype=torch.bfloat16)
    bias0 = (torch.randn(E, generator=gen) * 0.1).to(torch.bfloat16)
    with torch.no_grad():
        router.expert_bias_E.copy_(bias0)
    x = torch.randn(T, D, generator=gen).to(device=DEV, dtype=torch.bfloat16)
    w_DE = router.w_DE.detach()

    dt, st = dtype_code(torch.bfloat16), stream_of(DEV)
    EP = (E + 15) // 16 * 16
    EP = EP if EP <= 64 else (128 if EP <= 128 else (EP + 255) // 256 * 256)
    logits = torch.empty(T, E, dtype=torch.bfloat16, device=DEV)
    weights = torch.empty(T, K, dtype=torch.bfloat16, device=DEV)
    ind = torch.empty(T, K, dtype=torch.int64, device=DEV)
    idx32 = torch.empty(T, K, dtype=torch.int32, device=DEV)
    score = torch.empty(T, K, dtype=torch.float32, device=DEV)
    hist = torch.full((query("abacus_moe_hist_len", T, E),), -1, dtype=torch.int32, device=DEV)
    ws = torch.full((query("abacus_moe_router_ws_bytes", D, E, dt),), 0x7F, dtype=torch.uint8, device=DEV)
    call("abacus_moe_router_fwd", ptr(x), ptr(w_DE), ptr(router.expert_bias_E), T, D, E, K, 1.5, dt, ptr(logits),
         ptr(weights), ptr(ind), ptr(idx32), ptr(score), ptr(hist), ptr(ws), st)
    torch.cuda.synchronize()
    wt = ws[: EP * D * 2].view(torch.bfloat16).reshape(EP, D).cpu()
    want = torch.zeros(EP, D, dtype=torch.bfloat16)
    want[:E] = w_DE.t().cpu()
    assert torch.equal(wt, want)
    nb = (T + 15) // 16
    h = torch.zeros(nb, E, dtype=torch.int32)
    for t, row in enumerate(ind.cpu().tolist()):
        for e in row:
            h[t // 16, e] += 1
    assert torch.equal(hist.cpu().reshape(nb, E), h)

    xg = x.clone().requires_grad_()
    router.eval()
    w, idx = router(xg)
    torch.cuda.synchronize()
    lg = router.last_routing.logits_TE.cpu()
    assert torch.equal(lg, logits.cpu()) and torch.equal(idx, ind)
    w_o, idx_o, _ = oracle.route(lg, bias0, K, router.route_scale)
    assert torch.equal(idx.cpu(), idx_o)
    assert torch.equal(w.detach().cpu(), w_o)
    ref = (x.float() @ w_DE.float()).cpu()
    torch.testing.assert_close(lg.float(), ref, rtol=1e-2, atol=1e-2 * float(ref.std()))

    # Gradients against fp64 products with the kernel's own gating quantities (bf16 scores,
    # weights and rounded score sum in the formula of router.py:45,49-51: dL/dlogit_j =
    # (rho dw_j - sum_k dw_k w_k) / S * s_j (1 - s_j)), so the check is on the products with
    # w_DE (through the transposed copy) and x, not on bf16 rounding of saturated sigmoids.
    g = torch.randn(T, K, generator=gen)
    (w.float() * g.to(DEV)).sum().backward()
    sc, wk = score.cpu().double(), weights.cpu().double()
    dwk = g.to(torch.bfloat16).double()
    S = sc.sum(-1, keepdim=True).to(torch.bfloat16).double()
    dl = (1.5 * dwk - (dwk * wk).sum(-1, keepdim=True)) / S * sc * (1 - sc)
    G = torch.zeros(T, E, dtype=torch.float64).scatter_add_(1, ind.cpu(), dl)
    dx_ref = (G @ w_DE.cpu().double().t()).float()
    torch.testing.assert_close(xg.grad.float().cpu(), dx_ref, rtol=1e-2, atol=1e-2 * float(dx_ref.pow(2).mean().sqrt()))
    # dW = x^T G takes G as a bf16 operand (as bf16 autograd holds dlogits) and rounds once: per
    # element within 2^-9 of |x|^T |G| plus 2^-9 of the value, each allowed twice (where two
    # tokens' terms cancel, the operand rounding exceeds any tolerance relative to the value)
    xa = x.cpu().double()
    dw_ref = xa.t() @ G
    bound = 2.0**-8 * (xa.abs().t() @ G.abs() + dw_ref.abs())
    err = (router.w_DE.grad.double().cpu() - dw_ref).abs()
    assert bool((err <= bound).all()), float((err - bound).max())


def test_update_bias_explicit_indices():
    router = Router(4, 4, 2, bias_update_speed=0.5).to(DEV)
    idx = torch.tensor([[0, 1], [0, 2], [0, 1]], device=DEV)
    router.update_bias(idx)
    assert router.expert_bias_E.tolist() == [-0.5, -0.5, 0.5, 0.5]



@pytest.mark.parametrize("E,K,dtype", SPECIAL_CASES, ids=[f"E{e}_K{k}_{str(d)[6:]}" for e, k, d in SPECIAL_CASES])
def test_selection_order_special_values(E, K, dtype):
    """NaN, +-inf, exact ties and zero selections: see tests/special_selection.py."""
    print(f"\n[routing-special] E={E} K={K} {dtype}", flush=True)
    check_special_selection(E, K, dtype, DEV)


@pytest.mark.parametrize("E,K,T", LARGE_BATCH_CASES, ids=[f"E{e}_K{k}_T{t}" for e, k, t in LARGE_BATCH_CASES])
def test_selection_order_special_values_large_batch(E, K, T):
    """The same special selections through the bf16 router's 64-token blocks (T >= 8192)."""
    print(f"\n[routing-special-large] E={E} K={K} T={T}", flush=True)
    check_special_selection(E, K, torch.bfloat16, DEV, T=T)


@pytest.mark.parametrize("T,D,E,K,dtype", [(1, 64, 4, 2, torch.float32), (200, 128, 64, 6, torch.bfloat16),
                                           (4096, 256, 8, 2, torch.bfloat16), (3000, 64, 16, 4, torch.float32),
                                           (5000, 64, 16, 2, torch.bfloat16), (33, 72, 256, 16, torch.bfloat16),
                                           (64, 328, 64, 6, torch.bfloat16), (48, 1032, 16, 4, torch.float32),
                                           (64, 2048, 64, 6, torch.bfloat16),
                                           # more than 256 experts or 16 slots: scan and 64-slot gather
                                           (100, 64, 300, 20, torch.bfloat16), (40, 128, 1024, 64, torch.float32),
                                           (16, 64, 520, 7, torch.bfloat16), (70, 96, 48, 33, torch.float32)])
def test_dispatch_matches_scan_then_gather(T, D, E, K, dtype):
    """abacus_moe_dispatch (one launch when the block histograms hold at most 4096 ints: the gather
    blocks scan them) equals abacus_moe_route_scan + abacus_moe_permute_gather bit for bit:
    counts, offsets, pos, perm, the gathered rows and the bias step; counts, perm and the gathered
    rows (x[perm]) equal the oracle's."""
    from abacus_amd._lib import call, ptr, query, stream_of, dtype_code
    print(f"\n[dispatch] T={T} D={D} E={E} K={K} {dtype}", flush=True)
    gen = torch.Generator().manual_seed(T + E)
    router = Router(D, E, K).to(device=DEV, dtype=dtype)
    x = torch.randn(T, D, generator=gen).to(device=DEV, dtype=dtype)
    router.eval()
    with torch.no_grad():
        router(x)
    r = router.last_routing
    idx = r.indices_TK.to(torch.int32).contiguous()
    # the block histograms as the router kernel writes them: counts per 16-token block
    nb = (T + 15) // 16
    hist = torch.zeros(nb, E, dtype=torch.int32)
    for t, row in enumerate(idx.cpu().tolist()):
        for e in row:
            hist[t // 16, e] += 1
    hist = hist.to(DEV).reshape(-1).contiguous()
    assert hist.numel() == query("abacus_moe_hist_len", T, E)
    dt, s = dtype_code(dtype), stream_of(DEV)
    bias0 = (torch.randn(E, generator=gen) * 0.1).to(device=DEV, dtype=dtype)
    outs = []
    for fused in (False, True):
        bias = bias0.clone()
        counts = torch.full((E,), -1, dtype=torch.int32, device=DEV)
        offsets = torch.full((E + 1,), -1, dtype=torch.int32, device=DEV)
        pos = torch.full((T, K), -1, dtype=torch.int32, device=DEV)
        perm = torch.full((T * K,), -1, dtype=torch.int32, device=DEV)
        xp = torch.full((T * K, D), float("nan"), dtype=dtype, device=DEV)
        base = torch.full_like(hist, -1)
        if fused:
            call("abacus_moe_dispatch", ptr(hist), ptr(x), ptr(idx), T, D, E, K, ptr(bias), 0.25, dt, ptr(counts),
                 ptr(offsets), ptr(pos), ptr(perm), ptr(xp), ptr(base), s)
        else:
            call("abacus_moe_route_scan", ptr(hist), T, E, K, ptr(bias), 0.25, dt, ptr(base), ptr(counts),
                 ptr(offsets), s)
            call("abacus_moe_permute_gather", ptr(x), ptr(idx), ptr(base), T, D, E, K, dt, ptr(pos), ptr(perm),
                 ptr(xp), s)
        torch.cuda.synchronize()
        outs.append((counts.cpu(), offsets.cpu(), pos.cpu(), perm.cpu(), xp.cpu(), bias.cpu()))
    for name, a, b in zip(("counts", "offsets", "pos", "perm", "xp", "bias"), *outs):
        assert torch.equal(a, b), name
    counts_o, offsets_o, perm_o, pos_o = oracle.dispatch(idx.cpu().long(), E)
    assert outs[1][0].tolist() == counts_o.tolist() and outs[1][3].tolist() == perm_o.tolist()
    # the gathered rows themselves: small batches split each row over column chunks (at D = 328 bf16,
    # 41 vectors in 2 uneven chunks; at D = 1032 fp32, 258 vectors in 16 chunks, the last of 3)
    assert torch.equal(outs[1][4], x.cpu()[torch.as_tensor(perm_o, dtype=torch.long)])
