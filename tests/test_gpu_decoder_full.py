"""One training step of the full-size MoE decoder, in bf16 and in fp32 (transformer_moe.py:17-75, trainer.py:58-97):
8 layers, d_model 1024, 16 heads x 64 with RoPE and QK-norm, vocab 32000, an MoE FFN in every
layer (16 experts, top-2, SwiGLU hidden 2816), batch 4 x 2048.

Size-independent properties at the benchmark's own shape (the CPU restatement of the whole
decoder is too slow here; tests/test_gpu_transformer.py compares it at a reduced size): the HIP
flash-attention (bf16; fp32 attention runs torch's fused kernels), RMSNorm, MoE, cross-entropy and
AdamW entry points ran; the loss is finite and
close to ln(vocab) at initialisation; every layer's routing (indices, weights, the bias step) is
bit-exact against the oracle given that layer's logits; every parameter got a finite gradient
and every weight matrix moved.
"""

import math

import pytest
import torch

from abacus_amd import _lib
from abacus_amd.train import make_optimizer, train_step
from abacus.transformer_moe import TransformerMoe
from oracle import moe_oracle as oracle

pytestmark = pytest.mark.gpu

CFG = dict(dim=1024, n_heads=16, head_dim=64, n_blocks=8, vocab_size=32000, n_experts=16, top_k=2, hidden_dim=2816)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
def test_full_size_decoder_step(dtype):
    print(f"\n[decoder] full size, {dtype}, batch 4 x 2048", flush=True)
    torch.manual_seed(4)
    with torch.device("cuda"):  # initialised on the GPU: the values, not the host RNG stream, matter here
        model = TransformerMoe(**CFG)
    model = model.to(dtype)
    tokens = torch.randint(0, CFG["vocab_size"], (4, 2048), device="cuda")
    opt = make_optimizer(model)
    before = {n: p.detach().clone() for n, p in model.named_parameters()}
    bias0 = [b.moe.router.expert_bias_E.detach().clone() for b in model.blocks]
    timer = _lib.KernelTimer()
    with timer:
        loss = train_step(model, opt, tokens)
    calls = timer.totals_ms()
    wanted = ["abacus_rmsnorm_rope_fwd", "abacus_rmsnorm_rope_bwd", "abacus_rmsnorm_fwd", "abacus_rmsnorm_bwd",
              "abacus_moe_router_fwd", "abacus_moe_dispatch", "abacus_moe_gateup_fwd", "abacus_moe_down_fwd",
              "abacus_moe_combine_fwd", "abacus_moe_combine_bwd", "abacus_moe_down_bwd", "abacus_moe_gateup_bwd",
              "abacus_moe_unpermute_bwd", "abacus_moe_router_wgrad", "abacus_cross_entropy_fwd",
              "abacus_cross_entropy_bwd", "abacus_adamw_step"]
    if dtype == torch.bfloat16:
        wanted += ["abacus_attention_fwd", "abacus_attention_bwd"]
    for name in wanted:
        assert name in calls, f"{name} did not run"
    assert calls["abacus_moe_router_fwd"][1] == CFG["n_blocks"]
    assert math.isfinite(float(loss)) and abs(float(loss) - math.log(CFG["vocab_size"])) < 1.0

    K = CFG["top_k"]
    for i, (block, b0) in enumerate(zip(model.blocks, bias0)):
        r = block.moe.router.last_routing
        logits = r.logits_TE.cpu()
        w_o, idx_o, _ = oracle.route(logits, b0.cpu(), K, block.moe.router.route_scale)
        assert torch.equal(r.indices_TK.cpu(), idx_o), f"layer {i}: indices"
        assert torch.equal(r.weights_TK.cpu(), w_o), f"layer {i}: weights"
        stepped = oracle.bias_step(b0.cpu(), idx_o, CFG["n_experts"], block.moe.router.bias_update_speed)
        assert torch.equal(block.moe.router.expert_bias_E.cpu(), stepped), f"layer {i}: bias step"
        assert int(r.counts_E.sum()) == tokens.numel() * K

    for n, p in model.named_parameters():
        assert p.grad is not None and bool(torch.isfinite(p.grad).all()), f"{n}: gradient"
        # matrices move; a norm's gain of 1.0 may not (a 1e-3 step is below half a bf16 ulp there)
        if p.dim() >= 2:
            assert not torch.equal(p.detach(), before[n]), f"{n}: not updated"
