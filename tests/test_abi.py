"""The C ABI: libabacus_moe.so loads, exports every symbol include/abacus_moe.h declares,
the ctypes table matches the header, and argument validation fails cleanly (no GPU needed:
rejected calls return before any HIP call)."""

import ctypes
import pathlib
import re

import pytest
import torch

from abacus_amd import _lib

HEADER = pathlib.Path(__file__).resolve().parents[1] / "include" / "abacus_moe.h"


def _declarations():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    decls = {}
    for m in re.finditer(r"^\s*([A-Za-z_][\w\s\*]*?)\b(abacus_\w+)\s*\(([^;]*?)\)\s*;", text, flags=re.M | re.S):
        args = m.group(3).strip()
        n = 0 if args in ("", "void") else len(args.split(","))
        decls[m.group(2)] = n
    return decls


def test_header_declares_entry_points():
    decls = _declarations()
    assert len(decls) >= 20
    assert "abacus_moe_router_fwd" in decls and "abacus_moe_gateup_fwd" in decls


def test_ctypes_table_matches_header():
    decls = _declarations()
    assert set(decls) == set(_lib.SIGNATURES)
    for name, nargs in decls.items():
        assert len(_lib.SIGNATURES[name][1]) == nargs, name


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    for name in _declarations():
        assert hasattr(lib, name), name


def test_host_library_exports_its_entry_points():
    """libabacus_moe_host.so (CPU tensors) exports every MoE-layer, router and load-balancing entry
    point of the header, with the same ABI version."""
    lib = ctypes.CDLL(str(_lib.HOST_LIB_PATH))
    decls = _declarations()
    assert len(_lib.HOST_SYMBOLS) >= 25
    for name in _lib.HOST_SYMBOLS:
        assert name in decls and hasattr(lib, name), name
    assert _lib.load_host().abacus_moe_abi_version() == 5
    assert _lib.query("abacus_moe_hist_len", 4096, 8, device=torch.device("cpu")) == (4096 // 16) * 8


def test_abi_version_and_queries():
    lib = _lib.load()
    assert lib.abacus_moe_abi_version() == 5
    assert _lib.query("abacus_moe_hist_len", 4096, 8) == (4096 // 16) * 8
    assert _lib.query("abacus_moe_hist_len", 17, 8) == 2 * 8
    # bf16 with at most 256 experts: the transposed weight, then fp32 partial logits
    # (8 slices of D x 1024 tokens x padded experts) for the split small-batch router
    assert _lib.query("abacus_moe_router_ws_bytes", 4096, 8, _lib.BF16) == 16 * 4096 * 2 + 8 * 1024 * 16 * 4
    assert _lib.query("abacus_moe_router_ws_bytes", 4096, 128, _lib.BF16) == 128 * 4096 * 2 + 8 * 1024 * 128 * 4
    assert _lib.query("abacus_moe_router_ws_bytes", 4096, 128, _lib.F32) == 128 * 4096 * 4
    assert _lib.query("abacus_moe_router_ws_bytes", 1024, 17, _lib.F32) == 32 * 1024 * 4
    # past 256 experts the transposed weight has whole groups of 256 rows (the logits pass)
    assert _lib.query("abacus_moe_router_ws_bytes", 1024, 300, _lib.BF16) == 512 * 1024 * 2
    assert _lib.query("abacus_moe_router_ws_bytes", 512, 1024, _lib.F32) == 1024 * 512 * 4
    assert _lib.query("abacus_moe_router_wgrad_ws_bytes", 4096, 4096, 8, _lib.BF16) > 0
    assert _lib.query("abacus_moe_router_wgrad_ws_bytes", 4096, 4096, 8, 7) == -1
    # the down projection's split tail needs a workspace for long reductions (M >= 2560), none for
    # small batches or short reductions
    assert _lib.query("abacus_moe_down_fwd_ws_bytes", 8192, 14336, 4096, 8, _lib.BF16) > 0
    assert _lib.query("abacus_moe_down_fwd_ws_bytes", 16384, 2816, 1024, 16, _lib.BF16) > 0
    assert _lib.query("abacus_moe_down_fwd_ws_bytes", 16384, 2560, 1024, 16, _lib.F32) > 0
    assert _lib.query("abacus_moe_down_fwd_ws_bytes", 384, 1408, 2048, 64, _lib.BF16) == 0
    assert _lib.query("abacus_moe_down_fwd_ws_bytes", 65536, 768, 2048, 128, _lib.BF16) == 0
    assert _lib.query("abacus_moe_down_fwd_ws_bytes", 98304, 2559, 2048, 64, _lib.BF16) == 0
    assert _lib.query("abacus_attention_bwd_ws_bytes", 4, 2048, 16) == 4 * 16 * 2048 * 4


@pytest.mark.parametrize(
    "name,args,msg",
    [
        ("abacus_moe_router_fwd", (None, None, None, 16, 64, 1025, 2, 1.0, 1) + (None,) * 8, "n_experts"),
        ("abacus_moe_router_fwd", (None, None, None, 16, 64, 1024, 65, 1.0, 1) + (None,) * 8, "top_k"),
        ("abacus_moe_route_scan", (None, 16, 1025, 2, None, 0.0, 1, None, None, None, None), "n_experts"),
        ("abacus_router_gating_bwd", (None, None, None, 16, 65, 1.0, 1, None, None), "top_k"),
        ("abacus_moe_router_fwd", (None, None, None, 16, 64, 8, 9, 1.0, 1) + (None,) * 8, "top_k"),
        ("abacus_moe_permute_gather", (None, None, None, 16, 12, 8, 2, 1, None, None, None, None), "dim"),
        ("abacus_moe_router_fwd", (None, None, None, 16, 64, 8, 2, 1.0, 7) + (None,) * 8, "dtype"),
        ("abacus_moe_gateup_fwd", (None, None, None, None, 16, 64, 30, 8, 0, None, None, None, None), "hidden_dim"),
        ("abacus_moe_down_fwd", (None, None, None, 16, 64, 64, 0, 0, None, None, 0, None), "n_experts"),
        ("abacus_attention_fwd", (None, None, None, 1, 128, 1, 32, 0.125, 1, None, None, None), "head_dim"),
        ("abacus_attention_fwd", (None, None, None, 1, 100, 1, 64, 0.125, 1, None, None, None), "multiple of 128"),
        ("abacus_attention_fwd", (None, None, None, 1, 128, 1, 64, 0.125, 0, None, None, None), "bf16 only"),
        ("abacus_cross_entropy_fwd", (None, None, 4, 10, -100, 5, None, None, None), "dtype"),
        ("abacus_cross_entropy_bwd", (None, None, None, None, 1.0, 4, 0, -100, 1, None, None), "bad shape"),
        ("abacus_moe_gateup_bwd_wgrad", (None, None, None, None, 16, 64, 64, 8, 1, None, None, None, None),
         "tile_ctr"),
        ("abacus_moe_down_bwd", (None,) * 6 + (16, 64, 64, 8, 1) + (None,) * 5, "tile_ctr"),
    ],
)
def test_rejected_arguments_raise_with_message(name, args, msg):
    with pytest.raises(RuntimeError, match=msg):
        _lib.call(name, *args)
