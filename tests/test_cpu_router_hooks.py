"""Forward hooks on moe.router inside MoE.forward: the reference's MoE.forward calls self.router(x_BLD)
(moe.py:64), so hooks registered on the router see its input and its (weights_BLK, indices_BLK)
output (router.py:40-54).  The fused layer calls them with the routing it used; a hook that returns
a replacement raises NotImplementedError.  Host build (CPU tensors)."""

import pytest
import torch

from abacus.moe.moe import MoE


def _moe():
    torch.manual_seed(0)
    moe = MoE(16, 6, 2, hidden_dim=24, route_scale=1.5)
    with torch.no_grad():
        moe.router.w_DE.normal_(0.0, 0.5)
    return moe


def test_forward_and_pre_hooks_see_the_routing():
    moe = _moe()
    seen = []
    moe.router.register_forward_pre_hook(lambda m, args: seen.append(("pre", args[0].shape)))
    moe.router.register_forward_hook(lambda m, args, out: seen.append(("post", args[0].shape, out)))
    moe.router.register_forward_hook(lambda m, args, kwargs, out: seen.append(("kw", kwargs)), with_kwargs=True)
    x = torch.randn(3, 5, 16)
    moe.train()
    bias0 = moe.router.expert_bias_E.clone()
    moe(x)
    assert [s[0] for s in seen] == ["pre", "post", "kw"]
    assert seen[0][1] == x.shape and seen[1][1] == x.shape and seen[2][1] == {}
    w, idx = seen[1][2]
    r = moe.router.last_routing
    assert w.shape == (3, 5, 2) and idx.shape == (3, 5, 2) and idx.dtype == torch.int64
    assert torch.equal(idx.reshape(-1, 2), r.indices_TK) and torch.equal(w.reshape(-1, 2), r.weights_TK)
    # the same routing as the router module on its own, given the bias before this step
    with torch.no_grad():
        moe.router.expert_bias_E.copy_(bias0)
    moe.router.eval()
    w2, idx2 = moe.router(x)
    assert torch.equal(idx2, idx) and torch.equal(w2.detach(), w)


def test_empty_batch_still_calls_the_hooks():
    moe = _moe()
    seen = []
    moe.router.register_forward_hook(lambda m, args, out: seen.append(out))
    x = torch.randn(0, 4, 16)
    assert moe(x).shape == x.shape
    assert len(seen) == 1 and seen[0][0].shape == (0, 4, 2) and seen[0][1].shape == (0, 4, 2)


def test_hooks_that_replace_values_are_refused():
    moe = _moe()
    h = moe.router.register_forward_hook(lambda m, args, out: (out[0] * 2, out[1]))
    with pytest.raises(NotImplementedError, match="replace the router's output"):
        moe(torch.randn(2, 3, 16))
    h.remove()
    moe.router.register_forward_pre_hook(lambda m, args: (args[0] * 2,))
    with pytest.raises(NotImplementedError, match="replace the router's input"):
        moe(torch.randn(2, 3, 16))
