"""TransformerMoe (transformer_moe.py:17-75) on the GPU, MoE layers on the HIP path.

The same seeded model runs three ways: on the GPU, on the CPU in the same dtype,
and on the CPU in fp64 (the truth).  On the CPU each block's MoE is the oracle's
restatement, fed the routing the GPU chose so that a near-tie top-k cannot make
the runs diverge.  Criterion (as in test_gpu_moe.py): the GPU's normwise error
against fp64 is within twice the CPU's, or below the dtype's rtol (fp32 1e-5,
bf16 2e-2).
"""

import copy

import pytest
import torch
import torch.nn.functional as F

from abacus_amd import _lib
from abacus_amd.train import make_optimizer, train_step

from abacus.transformer_moe import TransformerMoe
from oracle import moe_oracle as oracle

pytestmark = pytest.mark.gpu

CFG = dict(dim=64, n_heads=4, head_dim=16, n_blocks=2, vocab_size=97, n_experts=4, top_k=2, hidden_dim=96)
RTOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2}


class _OracleMoE(torch.nn.Module):
    """CPU MoE from the oracle with fixed routing; shares the replaced module's parameters."""

    def __init__(self, moe, indices_TK):
        super().__init__()
        self.moe, self.indices = moe, indices_TK

    def forward(self, x_BLD):
        m = self.moe
        out, _ = oracle.moe_forward(
            x_BLD.reshape(-1, m.dim), m.router.w_DE, m.router.expert_bias_E, m.w_gate_EDM, m.w_up_EDM, m.w_down_EMD,
            m.top_k, m.router.route_scale, indices_TK=self.indices,
        )
        return out.reshape(x_BLD.shape)


def _run(model, tokens):
    logits = model(tokens)
    loss = F.cross_entropy(logits[:, :-1].reshape(-1, logits.shape[-1]).float(), tokens[:, 1:].reshape(-1))
    loss.backward()
    # the CPU models wrap each MoE once: blocks.i.moe.moe.* names the same parameter as blocks.i.moe.*
    grads = {n.replace(".moe.moe.", ".moe."): p.grad.detach().double().cpu()
             for n, p in model.named_parameters() if p.grad is not None}
    return logits.detach().double().cpu(), grads


def _rel(a, b):
    return float((a - b).norm() / max(b.norm().item(), 1e-30))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
def test_transformer_moe_matches_cpu_restatement(dtype):
    torch.manual_seed(4)
    base = TransformerMoe(**CFG).eval()
    tokens = torch.randint(0, CFG["vocab_size"], (2, 24))

    gpu = copy.deepcopy(base).to(dtype).cuda()
    got_logits, got_grads = _run(gpu, tokens.cuda())
    routes = [blk.moe.router.last_routing.indices_TK.detach().long().cpu() for blk in gpu.blocks]

    def cpu_model(dt):
        m = copy.deepcopy(base).to(dt)
        for blk, idx in zip(m.blocks, routes):
            blk.moe = _OracleMoE(blk.moe, idx)
        return m

    ref_logits, ref_grads = _run(cpu_model(dtype), tokens)
    tru_logits, tru_grads = _run(cpu_model(torch.float64), tokens)

    rtol = RTOL[dtype]
    e_gpu, e_cpu = _rel(got_logits, tru_logits), _rel(ref_logits, tru_logits)
    assert e_gpu <= max(2 * e_cpu, rtol), f"logits: gpu {e_gpu:.3g} vs cpu {e_cpu:.3g}"
    assert set(got_grads) == set(tru_grads)
    for name in tru_grads:
        e_gpu, e_cpu = _rel(got_grads[name], tru_grads[name]), _rel(ref_grads[name], tru_grads[name])
        assert e_gpu <= max(2 * e_cpu, rtol), f"{name}: gpu {e_gpu:.3g} vs cpu {e_cpu:.3g}"


def test_training_steps_reduce_loss_and_move_router_bias():
    torch.manual_seed(5)
    model = TransformerMoe(**CFG).to(torch.bfloat16).cuda().train()
    opt = make_optimizer(model, lr=3e-3)  # the reference's AdamW (HIP, one pass per tensor group)
    tokens = torch.randint(0, CFG["vocab_size"], (4, 32), device="cuda")
    tokens[1, 5:9] = -100  # padding: no embedding row, no target
    bias0 = [blk.moe.router.expert_bias_E.clone() for blk in model.blocks]
    losses = [float(train_step(model, opt, tokens)) for _ in range(8)]
    assert all(torch.isfinite(torch.tensor(losses)))
    assert losses[-1] < losses[0], losses
    assert any(not torch.equal(b0, blk.moe.router.expert_bias_E) for b0, blk in zip(bias0, model.blocks))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
@pytest.mark.parametrize("shape", [(2, 48, 4, 16), (1, 256, 2, 64)], ids=["L48_K16", "L256_K64"])
def test_attention_matches_materialised_fp64(dtype, shape):
    """MultiHeadAttention on the GPU (the HIP flash kernels for bf16 with head dim 64, torch's
    fused causal kernel elsewhere) against the materialised attention of attention.py:136-141
    in fp64."""
    from abacus_amd import transformer as tr
    B, L, H, K = shape
    torch.manual_seed(6)
    attn = tr.MultiHeadAttention(H * K, H, K)
    rot = tr.Rotary(K)
    x = torch.randn(B, L, H * K)

    def run(mod, xx, rotary):
        xx = xx.clone().requires_grad_()
        out = mod(xx, rotary)
        out.backward(torch.cos(torch.arange(out.numel(), dtype=out.dtype, device=out.device)).view_as(out))
        grads = [xx.grad] + [p.grad for p in mod.parameters()]
        return out.detach().double().cpu(), [g.detach().double().cpu() for g in grads]

    timer = _lib.KernelTimer()
    with timer:
        got, got_g = run(copy.deepcopy(attn).to(dtype).cuda(), x.to(dtype).cuda(),
                         copy.deepcopy(rot).to(dtype).cuda())
    calls = timer.totals_ms()
    ref, ref_g = run(copy.deepcopy(attn).to(dtype), x.to(dtype), copy.deepcopy(rot).to(dtype))
    tru, tru_g = run(copy.deepcopy(attn).double(), x.double(), copy.deepcopy(rot).double())
    rtol = RTOL[dtype]
    assert _rel(got, tru) <= max(2 * _rel(ref, tru), rtol)
    for g, r, t in zip(got_g, ref_g, tru_g):
        assert _rel(g, t) <= max(2 * _rel(r, t), rtol)
    if dtype == torch.bfloat16 and K == 64 and L % 128 == 0:
        # the HIP flash kernels take bf16, head dim 64, L a multiple of 128
        assert "abacus_attention_fwd" in calls and "abacus_attention_bwd" in calls, sorted(calls)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
@pytest.mark.parametrize("shape", [(2, 5, 1024), (3, 7, 4, 64), (1, 3, 2048), (1, 2, 512), (0, 4, 1024), (2, 3, 72)],
                         ids=["rows10_D1024", "rows84_D64", "D2048", "D512", "no_rows", "D72_fallback"])
def test_rmsnorm_matches_fp64(dtype, shape):
    """RMSNorm (norm.py:26-31) on the GPU -- the fused HIP kernel where it takes the
    shape -- against fp64: output, dx and dgamma; and bitwise repeatable."""
    from abacus_amd import transformer as tr
    torch.manual_seed(7)
    D = shape[-1]
    norm = tr.RMSNorm(D)
    with torch.no_grad():
        norm.w_gamma_D.copy_(1 + 0.1 * torch.randn(D))
    x = torch.randn(*shape)
    g = torch.randn(*shape)

    def run(mod, xx, gg):
        xx = xx.clone().requires_grad_()
        out = mod(xx)
        out.backward(gg)
        return [t.detach().double().cpu() for t in (out, xx.grad, mod.w_gamma_D.grad)]

    gpu_mod = copy.deepcopy(norm).to(dtype).cuda()
    got = run(gpu_mod, x.to(dtype).cuda(), g.to(dtype).cuda())
    again = run(copy.deepcopy(norm).to(dtype).cuda(), x.to(dtype).cuda(), g.to(dtype).cuda())
    ref = run(copy.deepcopy(norm).to(dtype), x.to(dtype), g.to(dtype))
    tru = run(copy.deepcopy(norm).double(), x.double(), g.double())
    rtol = RTOL[dtype]
    for name, a, b, r, t in zip(("y", "dx", "dgamma"), got, again, ref, tru):
        assert torch.equal(a, b), f"{name}: not bitwise repeatable"
        if t.numel() == 0 or t.norm() == 0:
            assert torch.count_nonzero(a) == 0
            continue
        assert _rel(a, t) <= max(2 * _rel(r, t), rtol), f"{name}: gpu {_rel(a, t):.3g} vs cpu {_rel(r, t):.3g}"
    assert tr._fused_norm_ok(x.to(dtype).cuda(), gpu_mod.w_gamma_D) == (D != 72)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
@pytest.mark.parametrize("shape", [(2, 9, 3, 64), (1, 33, 2, 16), (2, 5, 4, 128)], ids=["K64", "K16", "K128"])
def test_rmsnorm_rope_matches_fp64(dtype, shape):
    """The fused q/k norm + rotary kernel against RMSNorm then apply_rotary_pos_emb
    (norm.py:26-31, rope.py:36-46) in fp64: output, dx and dgamma."""
    from abacus_amd import transformer as tr
    B, L, H, K = shape
    torch.manual_seed(8)
    gamma = 1 + 0.1 * torch.randn(K)
    x = torch.randn(B, L, H, K)
    g = torch.randn(B, L, H, K)
    rot = tr.Rotary(K)
    cos, sin = rot(x, seq_dim=1)  # (1, 1, L, K) fp32

    def composite(xx, gm, c, s_):
        rms = torch.sqrt(xx.square().mean(-1, keepdim=True) + 1e-5)
        u = (gm * xx / rms).permute(0, 2, 1, 3)  # (B, H, L, K)
        out, _ = tr.apply_rotary_pos_emb(u, u, c, s_)
        return out.permute(0, 2, 1, 3)

    def run(fn, dev, dt):
        xx = x.detach().to(dev, dt).clone().requires_grad_()
        gm = gamma.detach().to(dev, dt).clone().requires_grad_()
        out = fn(xx, gm, cos.to(dev, dt), sin.to(dev, dt))
        out.backward(g.to(dev, dt))
        return [t.detach().double().cpu() for t in (out, xx.grad, gm.grad)]

    c_dev, s_dev = cos.to("cuda", dtype), sin.to("cuda", dtype)
    assert tr._fused_rope_ok(x.to("cuda", dtype), gamma.to("cuda", dtype), c_dev, s_dev)
    got = run(lambda xx, gm, c, s_: tr._RMSNormRopeFunction.apply(xx, gm, c.reshape(L, K), s_.reshape(L, K), 1e-5),
              "cuda", dtype)
    ref = run(composite, "cpu", dtype)
    tru = run(composite, "cpu", torch.float64)
    rtol = RTOL[dtype]
    for name, a, r, t in zip(("y", "dx", "dgamma"), got, ref, tru):
        assert _rel(a, t) <= max(2 * _rel(r, t), rtol), f"{name}: gpu {_rel(a, t):.3g} vs cpu {_rel(r, t):.3g}"


def test_trainer_step_matches_train_step():
    """abacus.trainer.Trainer(model).step (trainer.py:58-97, one process) is train_step with the
    reference's AdamW defaults: the same losses, parameters and moments over two steps; with
    total_steps the WSD rate is applied before each step."""
    from abacus.trainer import Trainer
    torch.manual_seed(23)
    model = TransformerMoe(vocab_size=512, dim=128, n_heads=2, head_dim=64, n_blocks=2, n_experts=4, top_k=2,
                           hidden_dim=256).to(torch.bfloat16).cuda()
    twin = copy.deepcopy(model)
    trainer = Trainer(model)
    opt = make_optimizer(twin)
    gen = torch.Generator().manual_seed(6)
    for _ in range(2):
        tokens = torch.randint(0, 512, (2, 128), generator=gen)
        tokens[0, 5] = -100
        loss, local = trainer.step(tokens)
        want = train_step(twin, opt, tokens.cuda())
        assert torch.equal(loss, want) and torch.equal(local, want)
    for (name, pa), pb in zip(model.named_parameters(), twin.parameters()):
        assert torch.equal(pa, pb), name
    scheduled = Trainer(copy.deepcopy(twin), total_steps=100)
    assert scheduled.optimizer.lr == scheduled.scheduler.learning_rate(1)
    scheduled.step(torch.randint(0, 512, (2, 128), generator=gen))
    assert scheduled.optimizer.lr == scheduled.scheduler.learning_rate(1)  # step 1 of 100: warmup 1/2


def test_liger_cross_entropy_matches_torch_on_gpu():
    """abacus.kernels.liger.cross_entropy on GPU logits: the HIP kernels with the row count kept
    on the device, against fp64; all rows ignored gives NaN, as torch's mean does."""
    from abacus.kernels.liger import cross_entropy
    g = torch.Generator(device="cuda").manual_seed(8)
    x = (torch.randn(500, 32000, device="cuda", generator=g) * 2).to(torch.bfloat16).requires_grad_()
    t = torch.randint(0, 32000, (500,), device="cuda", generator=g)
    t[::5] = -100
    loss = cross_entropy(x, t)
    (grad,) = torch.autograd.grad(loss, x)
    ref_x = x.detach().double().requires_grad_()
    ref = F.cross_entropy(ref_x, t)
    (ref_grad,) = torch.autograd.grad(ref, ref_x)
    assert loss.dtype == torch.bfloat16
    assert abs(float(loss.detach()) - float(ref.detach())) <= 2 ** -8 * abs(float(ref.detach()))
    assert float((grad.double() - ref_grad).norm() / ref_grad.norm()) < 4e-3
    assert torch.isnan(cross_entropy(x.detach(), torch.full_like(t, -100)))
    # options the kernels do not take go to torch's cross_entropy unchanged
    xd = x.detach()
    for kw in ({"label_smoothing": 0.1}, {"reduction": "sum"}, {"reduction": "none"}):
        torch.testing.assert_close(cross_entropy(xd, t, **kw), F.cross_entropy(xd, t, **kw), rtol=0, atol=0)
