"""ctypes binding of libabacus_moe.so (declarations in include/abacus_moe.h).

The HIP library is the only compute path for GPU tensors: if it is missing the
first call raises, there is no fallback.  CPU tensors go to libabacus_moe_host.so,
a host C++ build of the same entry points (abacus_amd/csrc/host/moe_host.cpp): a
call whose stream argument is stream_of(a CPU device) runs there.
"""

from __future__ import annotations

import ctypes
import pathlib
import threading

import torch

LIB_PATH = pathlib.Path(__file__).resolve().parent / "lib" / "libabacus_moe.so"
HOST_LIB_PATH = pathlib.Path(__file__).resolve().parent / "lib" / "libabacus_moe_host.so"

F32 = 0
BF16 = 1
F64 = 2  # the host library (CPU tensors) only
F16 = 3  # the host library (CPU tensors) only
TILE_CTR_INTS = 16  # ABACUS_MOE_TILE_CTR_INTS

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float
_D = ctypes.c_double

# name -> (restype, argtypes); must match include/abacus_moe.h
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "abacus_moe_last_error": (ctypes.c_char_p, []),
    "abacus_moe_abi_version": (_I, []),
    "abacus_moe_hist_len": (_I64, [_I64, _I64]),
    "abacus_moe_router_ws_bytes": (_I64, [_I64, _I64, _I]),
    "abacus_moe_router_wgrad_ws_bytes": (_I64, [_I64, _I64, _I64, _I]),
    "abacus_moe_down_fwd_ws_bytes": (_I64, [_I64, _I64, _I64, _I64, _I]),
    "abacus_moe_load_balancing_ws_bytes": (_I64, [_I64, _I64]),
    "abacus_moe_load_balancing_fwd": (_I, [_P, _P, _I64, _I64, _I64, _D, _I, _P, _P, _P, _P, _P, _P]),
    "abacus_moe_load_balancing_bwd": (_I, [_P, _P, _I64, _I64, _D, _I, _P, _P]),
    "abacus_moe_router_fwd": (
        _I,
        [_P, _P, _P, _I64, _I64, _I64, _I64, _D, _I, _P, _P, _P, _P, _P, _P, _P, _P],
    ),
    "abacus_moe_route_scan": (_I, [_P, _I64, _I64, _I64, _P, _D, _I, _P, _P, _P, _P]),
    "abacus_moe_permute_gather": (_I, [_P, _P, _P, _I64, _I64, _I64, _I64, _I, _P, _P, _P, _P]),
    "abacus_moe_dispatch": (_I, [_P, _P, _P, _I64, _I64, _I64, _I64, _P, _D, _I, _P, _P, _P, _P, _P, _P, _P]),
    "abacus_moe_gateup_fwd": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I, _P, _P, _P, _P]),
    "abacus_moe_down_fwd": (_I, [_P, _P, _P, _I64, _I64, _I64, _I64, _I, _P, _P, _I64, _P]),
    "abacus_moe_combine_fwd": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I, _P, _P]),
    "abacus_moe_combine_bwd": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _D, _I, _P, _P, _P]),
    "abacus_moe_down_bwd_dgrad": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I, _P, _P, _P]),
    "abacus_moe_down_bwd_wgrad": (_I, [_P, _P, _P, _I64, _I64, _I64, _I64, _I, _P, _P, _P]),
    "abacus_moe_gateup_bwd_dgrad": (_I, [_P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I, _P, _P]),
    "abacus_moe_gateup_bwd_wgrad": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I, _P, _P, _P, _P]),
    "abacus_moe_down_bwd": (_I, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I, _P, _P, _P, _P, _P]),
    "abacus_moe_gateup_bwd": (_I, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I, _P, _P, _P, _P, _P]),
    "abacus_moe_unpermute_bwd": (_I, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I, _P, _P]),
    "abacus_moe_router_wgrad": (_I, [_P, _P, _P, _I64, _I64, _I64, _I64, _I, _P, _P, _P]),
    "abacus_moe_router_wgrad_noalloc": (_I, [_P, _P, _P, _I64, _I64, _I64, _I64, _I, _P, _P]),
    "abacus_router_gating_bwd": (_I, [_P, _P, _P, _I64, _I64, _D, _I, _P, _P]),
    "abacus_router_update_bias": (_I, [_P, _I64, _I64, _D, _I, _P, _P]),
    "abacus_rmsnorm_fwd": (_I, [_P, _P, _I64, _I64, _F, _I, _P, _P, _P]),
    "abacus_rmsnorm_bwd_ws_bytes": (_I64, [_I64, _I64]),
    "abacus_rmsnorm_bwd": (_I, [_P, _P, _P, _P, _I64, _I64, _I, _P, _P, _P, _I64, _P]),
    "abacus_rmsnorm_rope_fwd": (_I, [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _F, _I, _P, _P, _P]),
    "abacus_rmsnorm_rope_bwd": (_I, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I, _P, _P, _P, _I64, _P]),
    "abacus_attention_fwd": (_I, [_P, _P, _P, _I64, _I64, _I64, _I64, _F, _I, _P, _P, _P]),
    "abacus_attention_bwd_ws_bytes": (_I64, [_I64, _I64, _I64]),
    "abacus_attention_bwd": (_I, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _F, _I, _P, _P, _P, _P, _I64,
                                  _P]),
    "abacus_cross_entropy_fwd": (_I, [_P, _P, _I64, _I64, _I64, _I, _P, _P, _P]),
    "abacus_cross_entropy_bwd": (_I, [_P, _P, _P, _P, _F, _I64, _I64, _I64, _I, _P, _P]),
    "abacus_adamw_step": (_I, [_P, _P, _P, _P, _P, _P, _I, _D, _D, _D, _D, _D, _I, _P]),
}

# Entry points of the HIP library that the host library also provides: the MoE layer, the router and
# the load-balancing loss (the decoder's RMSNorm, attention, cross-entropy and AdamW entry points are
# GPU-only; on the CPU those modules use torch).
HOST_SYMBOLS = [n for n in SIGNATURES if n.startswith("abacus_moe_") or n.startswith("abacus_router_")]

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None
_host_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load libabacus_moe.so once and declare every entry point's signature."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is not built: run `python -m abacus_amd.build` "
                    "(the MoE layer has no non-HIP implementation)"
                )
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def load_host() -> ctypes.CDLL:
    """Load libabacus_moe_host.so (the entry points for CPU tensors) once."""
    global _host_lib
    if _host_lib is not None:
        return _host_lib
    with _lock:
        if _host_lib is None:
            if not HOST_LIB_PATH.exists():
                raise RuntimeError(f"{HOST_LIB_PATH} is not built: run `python -m abacus_amd.build`")
            lib = ctypes.CDLL(str(HOST_LIB_PATH))
            for name in HOST_SYMBOLS:
                res, args = SIGNATURES[name]
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _host_lib = lib
    return _host_lib


class _HostStream:
    """The stream argument of a call on CPU tensors: routes the call to the host library."""

    def __repr__(self) -> str:
        return "<host>"


HOST = _HostStream()


class KernelTimer:
    """Records a pair of HIP events around every entry-point call made while active
    (or only around the calls of the entry points named in `only`).

    The events go to torch's current stream, which is the stream every entry
    point is launched on, so (end - start) is that call's device time.  Each
    event record is a packet of its own between two kernels and delays the
    next one by a few microseconds, so a timer that names only the kernel it
    needs perturbs the surrounding time least.
    """

    def __init__(self, only: set[str] | None = None) -> None:
        self.events: list[tuple[str, torch.cuda.Event, torch.cuda.Event]] = []
        self.only = only

    def wants(self, name: str) -> bool:
        return self.only is None or name in self.only

    def __enter__(self) -> "KernelTimer":
        global _timer
        _timer = self
        return self

    def __exit__(self, *exc) -> None:
        global _timer
        _timer = None

    def totals_ms(self) -> dict[str, tuple[float, int]]:
        """name -> (total milliseconds, number of calls); synchronises."""
        torch.cuda.synchronize()
        out: dict[str, tuple[float, int]] = {}
        for name, a, b in self.events:
            ms, n = out.get(name, (0.0, 0))
            out[name] = (ms + a.elapsed_time(b), n + 1)
        return out


_timer: KernelTimer | None = None


def call(name: str, *args) -> None:
    """Call an entry point that returns a status code; raise on failure.

    The last argument is the stream: stream_of(device) of the tensors' device.  HOST (a CPU
    device's) runs the host library's entry point instead of the HIP one."""
    if args and args[-1] is HOST:
        lib = load_host()
        rc = getattr(lib, name)(*args[:-1], None)
        if rc != 0:
            msg = lib.abacus_moe_last_error().decode(errors="replace")
            raise RuntimeError(f"{name} failed ({rc}): {msg}")
        return
    lib = load()
    timer = _timer if _timer is not None and _timer.wants(name) else None
    if timer is not None:
        start = torch.cuda.Event(enable_timing=True)
        start.record()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.abacus_moe_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed ({rc}): {msg}")
    if timer is not None:
        end = torch.cuda.Event(enable_timing=True)
        end.record()
        timer.events.append((name, start, end))


def query(name: str, *args, device: torch.device | None = None) -> int:
    """A sizing query, answered by the library that will run on `device` (the HIP one by default)."""
    lib = load_host() if device is not None and device.type == "cpu" else load()
    return int(getattr(lib, name)(*args))


def dtype_code(dtype: torch.dtype, device: torch.device | None = None) -> int:
    """The ABI dtype code.  float32 and bfloat16 run everywhere; float64 and float16 on CPU
    tensors only (the host library), and `device` other than the CPU refuses them."""
    if dtype == torch.float32:
        return F32
    if dtype == torch.bfloat16:
        return BF16
    if dtype in (torch.float64, torch.float16):
        if device is not None and device.type != "cpu":
            raise TypeError(f"abacus_amd's HIP kernels take float32 and bfloat16, got {dtype}; float64 and float16 "
                            "run on CPU tensors (the host library)")
        return F64 if dtype == torch.float64 else F16
    raise TypeError(f"abacus_amd MoE kernels support float32, bfloat16, and on CPU tensors float64 and float16; "
                    f"got {dtype}")


def acc_dtype(dtype: torch.dtype) -> torch.dtype:
    """The dtype of the fp32 side buffers (scores, dlogits, f_E): float64 for float64, else float32."""
    return torch.float64 if dtype == torch.float64 else torch.float32


def ptr(t: torch.Tensor | None) -> int | None:
    """Device address of a contiguous tensor (None -> NULL)."""
    if t is None:
        return None
    if not t.is_contiguous():
        raise ValueError("kernel operands must be contiguous")
    p = t.data_ptr()
    if p % 16 != 0 and t.numel() > 0:
        raise ValueError("kernel operands must be 16-byte aligned")
    return p


def tile_ctr(device: torch.device) -> torch.Tensor:
    """Tile-counter workspace of one weight-gradient call (the call clears it on its stream)."""
    return torch.empty(TILE_CTR_INTS, dtype=torch.int32, device=device)


def stream_of(device: torch.device):
    """The stream argument for a call on `device`'s tensors: torch's current HIP stream, or HOST."""
    if device.type == "cpu":
        return HOST
    return torch.cuda.current_stream(device).cuda_stream
