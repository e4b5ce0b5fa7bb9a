"""The combined backward GEMM entry points against the separate ones.

abacus_moe_down_bwd and abacus_moe_gateup_bwd run a data gradient and a weight
gradient in one launch (bf16) or as two launches (fp32, or shapes the pipelined
kernel does not take).  Either way their outputs must equal, bit for bit, what
the two single entry points produce on the same operands -- including experts
with no rows and a batch with no routed rows at all (the weight gradients are
then zeros and the data gradients empty).
"""

import itertools

import pytest
import torch

from abacus_amd import _lib

pytestmark = pytest.mark.gpu

call, ptr = _lib.call, _lib.ptr


def _operands(counts, D, M, dtype, seed):
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(seed)
    E, R = len(counts), sum(counts)
    offsets = torch.tensor([0] + list(itertools.accumulate(counts)), dtype=torch.int32, device=dev)

    def rn(*shape, scale=1.0):
        return (torch.randn(*shape, device=dev, generator=g) * scale).to(dtype)

    return dict(
        E=E, R=R, offsets=offsets,
        dy=rn(R, D), w_down=rn(E, M, D, scale=0.05), gate=rn(R, M), up=rn(R, M), h=rn(R, M),
        dgate=rn(R, M), dup=rn(R, M), w_gate=rn(E, D, M, scale=0.05), w_up=rn(E, D, M, scale=0.05), xp=rn(R, D),
    )


CASES = [
    # (counts per expert, D, M): bf16 takes the single pair launch, fp32 two launches
    ([300, 0, 500, 224], 256, 512),
    ([0, 0, 0, 0], 256, 512),
    ([1, 63, 0, 8], 128, 256),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("counts,D,M", CASES, ids=["ragged", "no_rows", "tiny"])
def test_down_bwd_pair_equals_separate_calls(dtype, counts, D, M):
    o = _operands(counts, D, M, dtype, seed=11)
    E, R, dt = o["E"], o["R"], _lib.dtype_code(dtype)
    dev = torch.device("cuda")
    s = _lib.stream_of(dev)
    out = {}
    for mode in ("pair", "single"):
        dg = torch.full((R, M), float("nan"), dtype=dtype, device="cuda")
        du = torch.full((R, M), float("nan"), dtype=dtype, device="cuda")
        dwd = torch.full((E, M, D), float("nan"), dtype=dtype, device="cuda")
        if mode == "pair":
            call("abacus_moe_down_bwd", ptr(o["dy"]), ptr(o["w_down"]), ptr(o["gate"]), ptr(o["up"]), ptr(o["h"]),
                 ptr(o["offsets"]), R, M, D, E, dt, ptr(dg), ptr(du), ptr(dwd), ptr(_lib.tile_ctr(dev)), s)
        else:
            call("abacus_moe_down_bwd_dgrad", ptr(o["dy"]), ptr(o["w_down"]), ptr(o["gate"]), ptr(o["up"]),
                 ptr(o["offsets"]), R, M, D, E, dt, ptr(dg), ptr(du), s)
            call("abacus_moe_down_bwd_wgrad", ptr(o["h"]), ptr(o["dy"]), ptr(o["offsets"]), R, M, D, E, dt,
                 ptr(dwd), ptr(_lib.tile_ctr(dev)), s)
        out[mode] = (dg, du, dwd)
    torch.cuda.synchronize()
    for a, b, name in zip(out["pair"], out["single"], ("dgate", "dup", "dw_down")):
        assert torch.equal(a, b), name
        assert not torch.isnan(a).any(), f"{name}: unwritten elements"
    # experts without rows get exactly zero weight gradient
    for e, c in enumerate(counts):
        if c == 0:
            assert torch.count_nonzero(out["pair"][2][e]) == 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
@pytest.mark.parametrize("counts,D,M", CASES, ids=["ragged", "no_rows", "tiny"])
def test_gateup_bwd_pair_equals_separate_calls(dtype, counts, D, M):
    o = _operands(counts, D, M, dtype, seed=12)
    E, R, dt = o["E"], o["R"], _lib.dtype_code(dtype)
    dev = torch.device("cuda")
    s = _lib.stream_of(dev)
    out = {}
    for mode in ("pair", "single"):
        dx = torch.full((R, D), float("nan"), dtype=dtype, device="cuda")
        dwg = torch.full((E, D, M), float("nan"), dtype=dtype, device="cuda")
        dwu = torch.full((E, D, M), float("nan"), dtype=dtype, device="cuda")
        if mode == "pair":
            call("abacus_moe_gateup_bwd", ptr(o["dgate"]), ptr(o["dup"]), ptr(o["w_gate"]), ptr(o["w_up"]),
                 ptr(o["xp"]), ptr(o["offsets"]), R, D, M, E, dt, ptr(dx), ptr(dwg), ptr(dwu),
                 ptr(_lib.tile_ctr(dev)), s)
        else:
            call("abacus_moe_gateup_bwd_dgrad", ptr(o["dgate"]), ptr(o["dup"]), ptr(o["w_gate"]), ptr(o["w_up"]),
                 ptr(o["offsets"]), R, D, M, E, dt, ptr(dx), s)
            call("abacus_moe_gateup_bwd_wgrad", ptr(o["xp"]), ptr(o["dgate"]), ptr(o["dup"]), ptr(o["offsets"]),
                 R, D, M, E, dt, ptr(dwg), ptr(dwu), ptr(_lib.tile_ctr(dev)), s)
        out[mode] = (dx, dwg, dwu)
    torch.cuda.synchronize()
    for a, b, name in zip(out["pair"], out["single"], ("dx_perm", "dw_gate", "dw_up")):
        assert torch.equal(a, b), name
        assert not torch.isnan(a).any(), f"{name}: unwritten elements"
    for e, c in enumerate(counts):
        if c == 0:
            assert torch.count_nonzero(out["pair"][1][e]) == 0
            assert torch.count_nonzero(out["pair"][2][e]) == 0


def test_pair_results_match_fp64_products():
    """The pair launch's outputs are the products they claim to be (bf16 operands, fp64 truth)."""
    counts, D, M = [300, 0, 500, 224], 256, 512
    o = _operands(counts, D, M, torch.bfloat16, seed=13)
    E, R = o["E"], o["R"]
    s = _lib.stream_of(torch.device("cuda"))
    dx = torch.empty(R, D, dtype=torch.bfloat16, device="cuda")
    dwg = torch.empty(E, D, M, dtype=torch.bfloat16, device="cuda")
    dwu = torch.empty(E, D, M, dtype=torch.bfloat16, device="cuda")
    call("abacus_moe_gateup_bwd", ptr(o["dgate"]), ptr(o["dup"]), ptr(o["w_gate"]), ptr(o["w_up"]), ptr(o["xp"]),
         ptr(o["offsets"]), R, D, M, E, 1, ptr(dx), ptr(dwg), ptr(dwu), ptr(_lib.tile_ctr(torch.device("cuda"))), s)
    torch.cuda.synchronize()
    off = o["offsets"].tolist()
    f = lambda t: t.double().cpu()
    for e in range(E):
        a, b = off[e], off[e + 1]
        want_dx = f(o["dgate"][a:b]) @ f(o["w_gate"][e]).T + f(o["dup"][a:b]) @ f(o["w_up"][e]).T
        want_dwg = f(o["xp"][a:b]).T @ f(o["dgate"][a:b])
        for got, want, name in ((dx[a:b], want_dx, "dx"), (dwg[e], want_dwg, "dw_gate")):
            if want.numel() == 0:
                continue
            err = (f(got) - want).norm() / max(want.norm().item(), 1e-30)
            assert err < 1e-2, f"expert {e} {name}: relative error {err:.3g}"


def test_down_fwd_split_tail():
    """Tiles past the GPU's whole rounds run as reduction slices plus a reduce kernel: same product.
    (The split runs for reductions of at least 2560; M = 2560 is the shortest.)"""
    counts, D, M = [1100, 950, 1030, 1010, 990, 1060, 1000, 1052], 4096, 2560
    o = _operands(counts, D, M, torch.bfloat16, seed=14)
    E, R = o["E"], o["R"]
    h, w_down = o["h"], torch.randn(E, M, D, device="cuda", generator=torch.Generator(device="cuda").manual_seed(3))
    w_down = (w_down * 0.05).to(torch.bfloat16)
    s = _lib.stream_of(torch.device("cuda"))
    ws_bytes = _lib.query("abacus_moe_down_fwd_ws_bytes", R, M, D, E, 1)
    assert ws_bytes > 0, "this shape has a partial last round on any GPU of up to 256 CUs"
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    outs = []
    for use_ws in (True, True, False):
        y = torch.full((R, D), float("nan"), dtype=torch.bfloat16, device="cuda")
        call("abacus_moe_down_fwd", ptr(h), ptr(w_down), ptr(o["offsets"]), R, M, D, E, 1, ptr(y),
             ptr(ws) if use_ws else None, ws_bytes if use_ws else 0, s)
        outs.append(y)
    torch.cuda.synchronize()
    split1, split2, whole = outs
    assert torch.equal(split1, split2), "repeated split calls differ"
    assert not torch.isnan(split1).any()
    # only the fp32 summation order differs: a few elements one bf16 rounding apart
    diff = (split1.float() - whole.float()).abs()
    assert float(diff.max()) <= 2 ** -7 * float(whole.float().abs().max())
    assert float((diff > 0).float().mean()) < 0.05
    off = o["offsets"].tolist()
    for e in range(E):
        a, b = off[e], off[e + 1]
        want = h[a:b].float() @ w_down[e].float()
        err = float((split1[a:b].float() - want).norm() / want.norm())
        assert err < 1e-2, f"expert {e}: relative error {err:.3g}"


@pytest.mark.parametrize("counts", [[256, 257, 383, 384, 385, 511, 512, 1, 128, 129, 0, 130],
                                    [1, 128, 0, 64, 129, 300, 7, 90]], ids=["large", "small_batch"])
def test_row_tiles_every_remainder_class(counts):
    """Row-grouped products for experts whose last rows fill a full tile, spill into one
    (remainder > 128 rows) or fit a thin 128-row tile (1..128 rows), plus empty and
    sub-128-row experts: every row written, each expert's rows equal to its fp64 product.
    The second case averages under 128 rows per expert, where the down projection's
    forward also runs thin tiles."""
    D, M = 256, 256
    o = _operands(counts, D, M, torch.bfloat16, seed=21)
    E, R = o["E"], o["R"]
    s = _lib.stream_of(torch.device("cuda"))
    dev = "cuda"
    nan = lambda *shape: torch.full(shape, float("nan"), dtype=torch.bfloat16, device=dev)
    G, U, H, Y = nan(R, M), nan(R, M), nan(R, M), nan(R, D)
    dG, dU, dX = nan(R, M), nan(R, M), nan(R, D)
    call("abacus_moe_gateup_fwd", ptr(o["xp"]), ptr(o["w_gate"]), ptr(o["w_up"]), ptr(o["offsets"]), R, D, M, E, 1,
         ptr(G), ptr(U), ptr(H), s)
    call("abacus_moe_down_fwd", ptr(o["h"]), ptr(o["w_down"]), ptr(o["offsets"]), R, M, D, E, 1, ptr(Y), None, 0, s)
    call("abacus_moe_down_bwd_dgrad", ptr(o["dy"]), ptr(o["w_down"]), ptr(o["gate"]), ptr(o["up"]),
         ptr(o["offsets"]), R, M, D, E, 1, ptr(dG), ptr(dU), s)
    call("abacus_moe_gateup_bwd_dgrad", ptr(o["dgate"]), ptr(o["dup"]), ptr(o["w_gate"]), ptr(o["w_up"]),
         ptr(o["offsets"]), R, D, M, E, 1, ptr(dX), s)
    torch.cuda.synchronize()
    for name, t in (("G", G), ("U", U), ("H", H), ("Y", Y), ("dG", dG), ("dU", dU), ("dX", dX)):
        assert not torch.isnan(t).any(), f"{name}: rows left unwritten"
    f = lambda t: t.double().cpu()
    off = o["offsets"].tolist()

    def close(got, want, what, tol=1e-2):
        err = float((f(got) - want).norm() / max(want.norm().item(), 1e-30))
        assert err < tol, f"{what}: relative error {err:.3g}"

    for e in range(E):
        a, b = off[e], off[e + 1]
        if a == b:
            continue
        close(G[a:b], f(o["xp"][a:b]) @ f(o["w_gate"][e]), f"G expert {e}")
        close(U[a:b], f(o["xp"][a:b]) @ f(o["w_up"][e]), f"U expert {e}")
        g, u = f(G[a:b]), f(U[a:b])
        close(H[a:b], g * torch.sigmoid(g) * u, f"H expert {e}")
        close(Y[a:b], f(o["h"][a:b]) @ f(o["w_down"][e]), f"Y expert {e}")
        dh = f(o["dy"][a:b]) @ f(o["w_down"][e]).T
        gg, uu = f(o["gate"][a:b]), f(o["up"][a:b])
        sg = torch.sigmoid(gg)
        close(dG[a:b], dh * uu * sg * (1 + gg * (1 - sg)), f"dG expert {e}", 2e-2)
        close(dU[a:b], dh * gg * sg, f"dU expert {e}", 2e-2)
        close(dX[a:b], f(o["dgate"][a:b]) @ f(o["w_gate"][e]).T + f(o["dup"][a:b]) @ f(o["w_up"][e]).T,
              f"dX expert {e}")


def test_fp32_row_products_at_pipelined_sizes():
    """fp32 row-grouped products with enough rows for the pipelined kernel (at least one round
    of 256 x 256 tiles per CU on a 256-CU GPU): every remainder class of an expert's last
    tile, an empty and a one-row expert, the down projection's forward with its split tail
    (a reduction of at least 2560) and without it, each expert's rows against the fp64 product
    (relative error 1e-5)."""
    base = [256, 257, 383, 384, 385, 511, 512, 1, 128, 129, 0, 130]
    counts = [c + (1536 if c > 1 else 0) for c in base] + [4000, 3000]
    D, M = 1024, 2560
    o = _operands(counts, D, M, torch.float32, seed=41)
    E, R = o["E"], o["R"]
    assert R >= 256 * 256 // (D // 256)
    s = _lib.stream_of(torch.device("cuda"))
    nan = lambda *shape: torch.full(shape, float("nan"), dtype=torch.float32, device="cuda")
    G, U, H, Y, Yw = nan(R, M), nan(R, M), nan(R, M), nan(R, D), nan(R, D)
    dG, dU, dX = nan(R, M), nan(R, M), nan(R, D)
    ws_bytes = _lib.query("abacus_moe_down_fwd_ws_bytes", R, M, D, E, 0)
    assert ws_bytes > 0, "this shape has a partial last round on any GPU of up to 256 CUs"
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
    call("abacus_moe_gateup_fwd", ptr(o["xp"]), ptr(o["w_gate"]), ptr(o["w_up"]), ptr(o["offsets"]), R, D, M, E, 0,
         ptr(G), ptr(U), ptr(H), s)
    call("abacus_moe_down_fwd", ptr(o["h"]), ptr(o["w_down"]), ptr(o["offsets"]), R, M, D, E, 0, ptr(Y), ptr(ws),
         ws_bytes, s)
    call("abacus_moe_down_fwd", ptr(o["h"]), ptr(o["w_down"]), ptr(o["offsets"]), R, M, D, E, 0, ptr(Yw), None, 0, s)
    call("abacus_moe_down_bwd_dgrad", ptr(o["dy"]), ptr(o["w_down"]), ptr(o["gate"]), ptr(o["up"]),
         ptr(o["offsets"]), R, M, D, E, 0, ptr(dG), ptr(dU), s)
    call("abacus_moe_gateup_bwd_dgrad", ptr(o["dgate"]), ptr(o["dup"]), ptr(o["w_gate"]), ptr(o["w_up"]),
         ptr(o["offsets"]), R, D, M, E, 0, ptr(dX), s)
    torch.cuda.synchronize()
    for name, t in (("G", G), ("U", U), ("H", H), ("Y", Y), ("Y whole", Yw), ("dG", dG), ("dU", dU), ("dX", dX)):
        assert not torch.isnan(t).any(), f"{name}: rows left unwritten"
    f = lambda t: t.double()  # fp64 products on the GPU: the CPU would take minutes at this size
    off = o["offsets"].tolist()

    def close(got, want, what):
        err = float((f(got) - want).norm() / max(want.norm().item(), 1e-30))
        assert err < 1e-5, f"{what}: relative error {err:.3g}"

    for e in range(E):
        a, b = off[e], off[e + 1]
        if a == b:
            continue
        close(G[a:b], f(o["xp"][a:b]) @ f(o["w_gate"][e]), f"G expert {e}")
        close(U[a:b], f(o["xp"][a:b]) @ f(o["w_up"][e]), f"U expert {e}")
        g, u = f(G[a:b]), f(U[a:b])
        close(H[a:b], g * torch.sigmoid(g) * u, f"H expert {e}")
        y = f(o["h"][a:b]) @ f(o["w_down"][e])
        close(Y[a:b], y, f"Y (split tail) expert {e}")
        close(Yw[a:b], y, f"Y (whole tiles) expert {e}")
        dh = f(o["dy"][a:b]) @ f(o["w_down"][e]).T
        gg, uu = f(o["gate"][a:b]), f(o["up"][a:b])
        sg = torch.sigmoid(gg)
        close(dG[a:b], dh * uu * sg * (1 + gg * (1 - sg)), f"dG expert {e}")
        close(dU[a:b], dh * gg * sg, f"dU expert {e}")
        close(dX[a:b], f(o["dgate"][a:b]) @ f(o["w_gate"][e]).T + f(o["dup"][a:b]) @ f(o["w_up"][e]).T,
              f"dX expert {e}")


def test_fp32_weight_gradients_at_pipelined_sizes():
    """fp32 weight gradients with enough per-expert tiles for the pipelined kernel (one block per
    tile, tile groups dealt to the XCDs in turn): skewed row counts with an empty and a one-row
    expert, each expert's dW against the fp64 product (relative error 1e-5), exact zeros for the
    empty expert, and the pair entry points equal to the single ones bit for bit."""
    counts = [3000, 1, 0, 700, 2500, 129, 1800, 64, 900, 4100, 333, 256, 1200, 40, 2000, 511]
    D, M = 1024, 1024
    o = _operands(counts, D, M, torch.float32, seed=43)
    E, R = o["E"], o["R"]
    assert E * (M // 256) * (D // 256) >= 256, "a round of down-projection weight-gradient tiles"
    dev = torch.device("cuda")
    s = _lib.stream_of(dev)
    nan = lambda *shape: torch.full(shape, float("nan"), dtype=torch.float32, device="cuda")
    dwd, dwg, dwu = nan(E, M, D), nan(E, D, M), nan(E, D, M)
    call("abacus_moe_down_bwd_wgrad", ptr(o["h"]), ptr(o["dy"]), ptr(o["offsets"]), R, M, D, E, 0, ptr(dwd),
         ptr(_lib.tile_ctr(dev)), s)
    call("abacus_moe_gateup_bwd_wgrad", ptr(o["xp"]), ptr(o["dgate"]), ptr(o["dup"]), ptr(o["offsets"]), R, D, M, E,
         0, ptr(dwg), ptr(dwu), ptr(_lib.tile_ctr(dev)), s)
    pdg, pdu, pdwd = nan(R, M), nan(R, M), nan(E, M, D)
    pdx, pdwg, pdwu = nan(R, D), nan(E, D, M), nan(E, D, M)
    call("abacus_moe_down_bwd", ptr(o["dy"]), ptr(o["w_down"]), ptr(o["gate"]), ptr(o["up"]), ptr(o["h"]),
         ptr(o["offsets"]), R, M, D, E, 0, ptr(pdg), ptr(pdu), ptr(pdwd), ptr(_lib.tile_ctr(dev)), s)
    call("abacus_moe_gateup_bwd", ptr(o["dgate"]), ptr(o["dup"]), ptr(o["w_gate"]), ptr(o["w_up"]), ptr(o["xp"]),
         ptr(o["offsets"]), R, D, M, E, 0, ptr(pdx), ptr(pdwg), ptr(pdwu), ptr(_lib.tile_ctr(dev)), s)
    torch.cuda.synchronize()
    for name, a, b in (("dw_down", dwd, pdwd), ("dw_gate", dwg, pdwg), ("dw_up", dwu, pdwu)):
        assert not torch.isnan(a).any(), f"{name}: unwritten elements"
        assert torch.equal(a, b), f"{name}: pair and single entry points differ"
    f = lambda t: t.double()
    off = o["offsets"].tolist()
    for e, c in enumerate(counts):
        a, b = off[e], off[e + 1]
        if c == 0:
            for name, t in (("dw_down", dwd), ("dw_gate", dwg), ("dw_up", dwu)):
                assert torch.count_nonzero(t[e]) == 0, f"{name}: expert {e} without rows"
            continue
        for name, got, want in (("dw_down", dwd[e], f(o["h"][a:b]).T @ f(o["dy"][a:b])),
                                ("dw_gate", dwg[e], f(o["xp"][a:b]).T @ f(o["dgate"][a:b])),
                                ("dw_up", dwu[e], f(o["xp"][a:b]).T @ f(o["dup"][a:b]))):
            err = float((f(got) - want).norm() / max(want.norm().item(), 1e-30))
            assert err < 1e-5, f"{name} expert {e}: relative error {err:.3g}"


WGRAD_CASES = [
    # (counts per expert, D, M): fewer tiles than CUs (most blocks find no tile), and more
    ([5, 0, 300, 64], 256, 256),
    ([700, 0, 1500, 64, 1030, 0], 1024, 2048),
]


def _wgrads(o, D, M, s, out=None, ctrs=None):
    """Both weight gradients through the single entry points (persistent tile loop), into `out` or new buffers.

    ctrs: the two calls' tile-counter workspaces (fresh ones when None); the caller keeps them alive
    until the calls are done."""
    E, R = o["E"], o["R"]
    if out is None:
        out = tuple(torch.full(shape, float("nan"), dtype=torch.bfloat16, device="cuda")
                    for shape in ((E, M, D), (E, D, M), (E, D, M)))
    if ctrs is None:
        ctrs = (_lib.tile_ctr(torch.device("cuda")), _lib.tile_ctr(torch.device("cuda")))
    dwd, dwg, dwu = out
    call("abacus_moe_down_bwd_wgrad", ptr(o["h"]), ptr(o["dy"]), ptr(o["offsets"]), R, M, D, E, 1, ptr(dwd),
         ptr(ctrs[0]), s)
    call("abacus_moe_gateup_bwd_wgrad", ptr(o["xp"]), ptr(o["dgate"]), ptr(o["dup"]), ptr(o["offsets"]), R, D, M, E,
         1, ptr(dwg), ptr(dwu), ptr(ctrs[1]), s)
    return out


@pytest.mark.parametrize("counts,D,M", WGRAD_CASES, ids=["few_tiles", "many_tiles"])
def test_wgrad_tile_loop(counts, D, M):
    """Weight gradients from the persistent tile loop: each expert's product (fp64 truth), exact
    zeros for experts without rows, bit-identical results over 70 launches that reuse one
    counter workspace left dirty by the previous launch (or filled with junk: each call clears
    its own), and with launches in flight on two streams at once, each with its own workspace."""
    o = _operands(counts, D, M, torch.bfloat16, seed=31)
    dev = torch.device("cuda")
    s = _lib.stream_of(dev)
    first = _wgrads(o, D, M, s)
    torch.cuda.synchronize()
    for name, t in zip(("dw_down", "dw_gate", "dw_up"), first):
        assert not torch.isnan(t).any(), f"{name}: unwritten elements"
    f = lambda t: t.double().cpu()
    off = o["offsets"].tolist()
    for e, c in enumerate(counts):
        a, b = off[e], off[e + 1]
        if c == 0:
            for t in first:
                assert torch.count_nonzero(t[e]) == 0
            continue
        for got, want, name in ((first[0][e], f(o["h"][a:b]).T @ f(o["dy"][a:b]), "dw_down"),
                                (first[1][e], f(o["xp"][a:b]).T @ f(o["dgate"][a:b]), "dw_gate"),
                                (first[2][e], f(o["xp"][a:b]).T @ f(o["dup"][a:b]), "dw_up")):
            err = float((f(got) - want).norm() / want.norm())
            assert err < 1e-2, f"expert {e} {name}: relative error {err:.3g}"
    # 70 launches of each kind on one stream, same buffers and the same two counter workspaces
    again = tuple(torch.empty_like(t) for t in first)
    ctrs = (_lib.tile_ctr(dev), _lib.tile_ctr(dev))
    for i in range(70):
        for t in again:
            t.fill_(float("nan"))
        if i % 10 == 0:
            for c in ctrs:
                c.fill_(123456 if i % 20 == 0 else -7)
        _wgrads(o, D, M, s, again, ctrs)
        torch.cuda.synchronize()
        for a, b, name in zip(first, again, ("dw_down", "dw_gate", "dw_up")):
            assert torch.equal(a, b), f"launch {i + 1}: {name} differs"
    # two streams (default priority) with launches in flight on both at once
    streams = [torch.cuda.Stream(device=dev), torch.cuda.Stream(device=dev)]
    outs = [tuple(torch.full_like(t, float("nan")) for t in first) for _ in range(6)]
    wss = [(_lib.tile_ctr(dev), _lib.tile_ctr(dev)) for _ in outs]
    torch.cuda.synchronize()
    for i, out in enumerate(outs):
        _wgrads(o, D, M, streams[i % 2].cuda_stream, out, wss[i])
    torch.cuda.synchronize()
    for i, out in enumerate(outs):
        for a, b, name in zip(first, out, ("dw_down", "dw_gate", "dw_up")):
            assert torch.equal(a, b), f"stream launch {i}: {name} differs"


def test_one_expert_dense_products():
    """All rows on one expert (the MoE layer with E = 1, a dense SwiGLU block; bench.py --gemm-shapes
    times it): many full row tiles and a remainder, a down projection long enough for its split tail,
    and weight gradients reducing over every row (one expert's few output tiles, each hundreds of
    k-tiles long). Every product of the four entry points against fp64."""
    counts, D, M = [4100], 512, 2816
    o = _operands(counts, D, M, torch.bfloat16, seed=41)
    E, R = o["E"], o["R"]
    dev = torch.device("cuda")
    s = _lib.stream_of(dev)
    nan = lambda *shape: torch.full(shape, float("nan"), dtype=torch.bfloat16, device="cuda")
    G, U, H, Y = nan(R, M), nan(R, M), nan(R, M), nan(R, D)
    dG, dU, dX = nan(R, M), nan(R, M), nan(R, D)
    dWd, dWg, dWu = nan(E, M, D), nan(E, D, M), nan(E, D, M)
    ws_bytes = _lib.query("abacus_moe_down_fwd_ws_bytes", R, M, D, E, 1)
    ws = torch.empty(max(ws_bytes, 16), dtype=torch.uint8, device="cuda")
    call("abacus_moe_gateup_fwd", ptr(o["xp"]), ptr(o["w_gate"]), ptr(o["w_up"]), ptr(o["offsets"]), R, D, M, E, 1,
         ptr(G), ptr(U), ptr(H), s)
    call("abacus_moe_down_fwd", ptr(o["h"]), ptr(o["w_down"]), ptr(o["offsets"]), R, M, D, E, 1, ptr(Y), ptr(ws),
         ws_bytes, s)
    call("abacus_moe_down_bwd", ptr(o["dy"]), ptr(o["w_down"]), ptr(o["gate"]), ptr(o["up"]), ptr(o["h"]),
         ptr(o["offsets"]), R, M, D, E, 1, ptr(dG), ptr(dU), ptr(dWd), ptr(_lib.tile_ctr(dev)), s)
    call("abacus_moe_gateup_bwd", ptr(o["dgate"]), ptr(o["dup"]), ptr(o["w_gate"]), ptr(o["w_up"]), ptr(o["xp"]),
         ptr(o["offsets"]), R, D, M, E, 1, ptr(dX), ptr(dWg), ptr(dWu), ptr(_lib.tile_ctr(dev)), s)
    torch.cuda.synchronize()
    for name, t in (("G", G), ("U", U), ("H", H), ("Y", Y), ("dG", dG), ("dU", dU), ("dX", dX), ("dW_down", dWd),
                    ("dW_gate", dWg), ("dW_up", dWu)):
        assert not torch.isnan(t).any(), f"{name}: elements left unwritten"
    f = lambda t: t.double().cpu()

    def close(got, want, what, tol=1e-2):
        err = float((f(got) - want).norm() / want.norm())
        assert err < tol, f"{what}: relative error {err:.3g}"

    x, wg, wu, wd = f(o["xp"]), f(o["w_gate"][0]), f(o["w_up"][0]), f(o["w_down"][0])
    close(G, x @ wg, "G")
    close(U, x @ wu, "U")
    g, u = f(G), f(U)
    close(H, g * torch.sigmoid(g) * u, "H")
    close(Y, f(o["h"]) @ wd, "Y")
    dh = f(o["dy"]) @ wd.T
    gg, uu = f(o["gate"]), f(o["up"])
    sg = torch.sigmoid(gg)
    close(dG, dh * uu * sg * (1 + gg * (1 - sg)), "dG", 2e-2)
    close(dU, dh * gg * sg, "dU", 2e-2)
    close(dWd[0], f(o["h"]).T @ f(o["dy"]), "dW_down")
    close(dX, f(o["dgate"]) @ wg.T + f(o["dup"]) @ wu.T, "dX")
    close(dWg[0], x.T @ f(o["dgate"]), "dW_gate")
    close(dWu[0], x.T @ f(o["dup"]), "dW_up")
