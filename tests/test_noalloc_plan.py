"""Host-side logic of abacus_moe_router_wgrad_noalloc, without a GPU: the size check uses the
same partial-sum plan as the launch (its accept/reject boundary equals the per-dtype workspace
query over a grid of shapes), and the per-device scratch-address cache behaves for device indices
past 63 and under concurrent callers (tests/native/device_table_check.cpp, built with g++).

Rejected calls return before any HIP call, so they are safe on any machine; accepted calls are
made only where no GPU is visible, where they stop at the device lookup."""

import pathlib
import re
import shutil
import subprocess

import pytest
import torch

from abacus_amd import _lib
from abacus_amd._lib import call, query

ROOT = pathlib.Path(__file__).resolve().parents[1]
SCRATCH_BYTES = 32 << 20


def _noalloc_shape_only(T, D, E, K, dt):
    call("abacus_moe_router_wgrad_noalloc", None, None, None, T, D, E, K, dt, None, None)


def test_fp32_wide_path_beyond_the_scratch_is_rejected():
    """fp32, E = 64 runs the wide column kernel: at T = 16384, D = 2048 its plan has 128 token chunks,
    64 MiB of partial sums, twice the scratch (a plan for the register kernel would count 64 chunks
    and let it through)."""
    need = query("abacus_moe_router_wgrad_ws_bytes", 16384, 2048, 64, _lib.F32)
    assert need == 128 * 64 * 2048 * 4
    with pytest.raises(RuntimeError, match=f"needs {need} bytes.*static scratch"):
        _noalloc_shape_only(16384, 2048, 64, 6, _lib.F32)


GRID = [(T, D, E, dt) for T in (1, 100, 4096, 8192, 16384, 65536) for D in (512, 2048, 4096, 8192)
        for E in (8, 16, 32, 64, 256) for dt in (_lib.F32, _lib.BF16)]


def test_size_check_boundary_matches_the_workspace_query():
    """Over the grid, noalloc rejects exactly the shapes whose per-dtype workspace query exceeds the
    32 MiB scratch, and names that query's byte count in the message."""
    no_gpu = torch.cuda.device_count() == 0
    rejected = accepted = 0
    for T, D, E, dt in GRID:
        need = query("abacus_moe_router_wgrad_ws_bytes", T, D, E, dt)
        assert need > 0 and need % (E * D * 4) == 0
        if need > SCRATCH_BYTES:
            with pytest.raises(RuntimeError, match=f"needs {need} bytes.*static scratch"):
                _noalloc_shape_only(T, D, E, 2, dt)
            rejected += 1
        elif no_gpu:
            with pytest.raises(RuntimeError) as err:
                _noalloc_shape_only(T, D, E, 2, dt)
            assert "static scratch" not in str(err.value)
            assert re.search(r"HIP device|hipStreamGetDevice|hipGetSymbolAddress", str(err.value))
            accepted += 1
    assert rejected >= 20
    assert accepted >= 20 or not no_gpu


def test_workspace_query_rejects_unknown_dtype():
    assert query("abacus_moe_router_wgrad_ws_bytes", 4096, 4096, 8, 5) == -1


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not found")
def test_per_device_scratch_address_cache(tmp_path):
    exe = tmp_path / "device_table_check"
    src = ROOT / "tests" / "native" / "device_table_check.cpp"
    subprocess.run(["g++", "-O1", "-std=c++17", "-pthread", f"-I{ROOT / 'abacus_amd' / 'csrc'}", str(src), "-o",
                    str(exe)], check=True, capture_output=True, text=True)
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert res.returncode == 0 and res.stdout.strip() == "ok", res.stdout + res.stderr
