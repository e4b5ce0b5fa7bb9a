"""abacus_moe_router_wgrad_noalloc: the router weight gradient with its partial sums in the
library's static device scratch instead of a caller workspace.  Through the C ABI, its output
equals abacus_moe_router_wgrad's bit for bit, on two calls in a row (the second on a smaller
input, so the scratch still holds the first call's partials), on each of the three partial
kernels: bf16 with D a multiple of 8 (matrix-core kernel), fp32 with E <= 16 (register kernel),
fp32 with E > 16 (wide column kernel, including shapes whose partial sums fill the 32 MiB scratch
exactly); a shape whose partial sums exceed the scratch is rejected before any launch."""

import pytest
import torch

from abacus_amd import _lib
from abacus_amd._lib import call, ptr, query

DEV = torch.device("cuda", 0)


def _inputs(T, D, E, K, dtype, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn(T, D, device=DEV, generator=g).to(dtype)
    dlogit = torch.randn(T, K, device=DEV, generator=g)
    idx = torch.stack([torch.randperm(E, device=DEV, generator=g)[:K] for _ in range(T)]).to(torch.int32)
    return x, dlogit, idx.contiguous()


def _with_workspace(x, dlogit, idx, E):
    T, D = x.shape
    K = idx.shape[1]
    nbytes = query("abacus_moe_router_wgrad_ws_bytes", T, D, E, _lib.dtype_code(x.dtype))
    ws = torch.empty(nbytes // 4 + 1, dtype=torch.float32, device=DEV)
    dw = torch.full((D, E), float("nan"), dtype=x.dtype, device=DEV)
    call("abacus_moe_router_wgrad", ptr(x), ptr(dlogit), ptr(idx), T, D, E, K, _lib.dtype_code(x.dtype), ptr(ws),
         ptr(dw), _lib.stream_of(DEV))
    return dw


def _noalloc(x, dlogit, idx, E):
    T, D = x.shape
    K = idx.shape[1]
    dw = torch.full((D, E), float("nan"), dtype=x.dtype, device=DEV)
    call("abacus_moe_router_wgrad_noalloc", ptr(x), ptr(dlogit), ptr(idx), T, D, E, K, _lib.dtype_code(x.dtype),
         ptr(dw), _lib.stream_of(DEV))
    return dw


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("T,D,E,K,T2", [(4096, 4096, 8, 2, 1000), (8192, 1024, 16, 2, 333), (2048, 2048, 64, 6, 100)],
                         ids=["mixtral", "decoder", "skewed_E64"])
def test_noalloc_equals_workspace_entry_point(dtype, T, D, E, K, T2):
    print(f"\n[noalloc] T={T} then {T2} D={D} E={E} K={K} {dtype}", flush=True)
    for n, seed in ((T, 1), (T2, 2)):
        x, dlogit, idx = _inputs(n, D, E, K, dtype, seed)
        got = _noalloc(x, dlogit, idx, E)
        want = _with_workspace(x, dlogit, idx, E)
        torch.cuda.synchronize()
        assert not torch.isnan(want).any()
        assert torch.equal(got, want), f"T={n}: noalloc differs from the workspace entry point"


@pytest.mark.gpu
@pytest.mark.parametrize("T,D,E,K,T2", [(8192, 2048, 64, 6, 3000), (8192, 2048, 32, 4, 1500)],
                         ids=["E64_full_scratch", "E32_full_scratch"])
def test_noalloc_fp32_wide_path_at_the_scratch_limit(T, D, E, K, T2):
    """fp32 with E > 16 (the wide column kernel) at shapes whose partial sums are exactly 32 MiB."""
    assert query("abacus_moe_router_wgrad_ws_bytes", T, D, E, _lib.F32) == 32 << 20
    print(f"\n[noalloc] fp32 wide T={T} then {T2} D={D} E={E} K={K}", flush=True)
    for n, seed in ((T, 3), (T2, 4)):
        x, dlogit, idx = _inputs(n, D, E, K, torch.float32, seed)
        got = _noalloc(x, dlogit, idx, E)
        want = _with_workspace(x, dlogit, idx, E)
        torch.cuda.synchronize()
        assert not torch.isnan(want).any()
        assert torch.equal(got, want), f"T={n}: noalloc differs from the workspace entry point"


def test_noalloc_rejects_shapes_beyond_the_scratch():
    """E = 64, D = 262144: one token chunk of partial sums is 64 MiB, twice the scratch."""
    with pytest.raises(RuntimeError, match="static scratch"):
        call("abacus_moe_router_wgrad_noalloc", None, None, None, 64, 262144, 64, 2, _lib.BF16, None, None)
