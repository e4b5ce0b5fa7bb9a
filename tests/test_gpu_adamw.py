"""abacus_adamw_step and abacus_amd.optim.AdamW on the GPU.

The kernel must equal, bit for bit, the oracle's restatement of the reference's AdamW
(optimizers/adamw.py:85-119, every intermediate rounded to the parameter dtype) and the
reference's own tensor-op sequence run by torch on the GPU, over several steps, for more
tensors than one launch takes, sizes that are not whole 16-byte vectors, an empty tensor,
and parameters whose step counts differ (one without a gradient in a step is skipped).
"""

import numpy as np
import pytest
import torch

from abacus_amd import _lib
from abacus_amd.optim import AdamW
from oracle.adamw_oracle import adamw_step

pytestmark = pytest.mark.gpu

HP = dict(lr=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=1e-2)
SIZES = [4096, 1, 7, 8, 9, 1000, 0, 12345, 65536 + 3] + [37 * k + 5 for k in range(55)]  # 64 tensors


def _reference_ops(p, g, m, v, step, lr, beta1, beta2, eps, weight_decay):
    """adamw.py:104-119 as torch tensor ops (in place)."""
    if weight_decay != 0:
        p.mul_(1 - lr * weight_decay)
    m.lerp_(g, 1 - beta1)
    v.mul_(beta2).addcmul_(g, g, value=1 - beta2)
    bc1 = 1 - beta1 ** step
    bc2 = 1 - beta2 ** step
    denom = v.sqrt().div_(bc2 ** 0.5).add_(eps)
    p.addcdiv_(m, denom, value=-(lr / bc1))


class _Params(torch.nn.Module):
    def __init__(self, dtype):
        super().__init__()
        g = torch.Generator().manual_seed(7)
        self.ps = torch.nn.ParameterList(
            [torch.nn.Parameter((torch.randn(n, generator=g) * 0.5).to(dtype).cuda()) for n in SIZES])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
def test_adamw_matches_oracle_and_reference_ops(dtype):
    model = _Params(dtype)
    opt = AdamW(model, **{"lr": HP["lr"], "betas": (HP["beta1"], HP["beta2"]), "eps": HP["eps"],
                          "weight_decay": HP["weight_decay"]})
    params = list(model.parameters())
    ref = [[p.detach().clone(), torch.zeros_like(p), torch.zeros_like(p), 0] for p in params]  # torch ops
    ora = [[p.detach().float().cpu().numpy(), np.zeros(p.numel(), np.float32), np.zeros(p.numel(), np.float32), 0]
           for p in params]
    name = "bf16" if dtype == torch.bfloat16 else "fp32"
    gen = torch.Generator(device="cuda").manual_seed(11)
    for step in range(4):
        for i, p in enumerate(params):
            # step 1 leaves every third parameter without a gradient: its step count falls behind
            if step == 1 and i % 3 == 0:
                p.grad = None
                continue
            p.grad = (torch.randn(p.shape, device="cuda", generator=gen) * 10.0 ** (step - 2)).to(dtype)
        opt.step()
        for i, p in enumerate(params):
            if p.grad is None:
                continue
            r, o = ref[i], ora[i]
            r[3] += 1
            o[3] += 1
            _reference_ops(r[0], p.grad, r[1], r[2], r[3], **HP)
            o[0], o[1], o[2] = adamw_step(o[0], p.grad.float().cpu().numpy(), o[1], o[2], o[3], dtype=name, **HP)
        torch.cuda.synchronize()
        for i, p in enumerate(params):
            st = opt.state.get(id(p))
            if st is None:
                continue
            assert st["step"] == ora[i][3]
            for got, r_t, o_a, what in ((p.detach(), ref[i][0], ora[i][0], "param"),
                                        (st["exp_avg"], ref[i][1], ora[i][1], "exp_avg"),
                                        (st["exp_avg_sq"], ref[i][2], ora[i][2], "exp_avg_sq")):
                g_np = got.float().cpu().numpy()
                assert np.array_equal(g_np, o_a), f"step {step} tensor {i} ({SIZES[i]}): {what} != oracle"
                assert torch.equal(got, r_t), f"step {step} tensor {i} ({SIZES[i]}): {what} != torch ops"
    assert opt.state[id(params[0])]["step"] == 3 and opt.state[id(params[1])]["step"] == 4


def test_adamw_api_errors_and_state_layout():
    model = torch.nn.Linear(16, 8).cuda()
    with pytest.raises(ValueError, match="Invalid learning rate"):
        AdamW(model, lr=-1.0)
    with pytest.raises(ValueError, match="Invalid epsilon"):
        AdamW(model, eps=-1.0)
    with pytest.raises(ValueError, match="Invalid betas"):
        AdamW(model, betas=(1.0, 0.9))
    with pytest.raises(ValueError, match="Invalid weight decay"):
        AdamW(model, weight_decay=-0.1)
    opt = AdamW(model)
    opt.step()  # no gradients: nothing changes, no state
    assert opt.state == {}
    model(torch.randn(4, 16, device="cuda")).sum().backward()
    w0 = model.weight.detach().clone()
    opt.step()
    st = opt.state[id(model.weight)]
    assert st["step"] == 1 and st["exp_avg"].shape == model.weight.shape
    assert st["exp_avg"].dtype == model.weight.dtype and not torch.equal(model.weight, w0)
    opt.zero_grad()
    assert all(p.grad is None for p in model.parameters())
    # the entry point rejects bad arguments before launching anything
    with pytest.raises(RuntimeError, match="invalid hyperparameters"):
        _lib.call("abacus_adamw_step", None, None, None, None, None, None, 0, 1e-3, 1.5, 0.999, 1e-8, 0.0, 1,
                  _lib.stream_of(torch.device("cuda")))
