"""Build recipe for libabacus_moe.so (the MI355X / gfx950 MoE kernel library) and
libabacus_moe_host.so (the same C ABI built for CPU tensors).

Compiles every ``abacus_amd/csrc/*.hip`` translation unit with hipcc for
gfx950 and links them into ``abacus_amd/lib/libabacus_moe.so`` in-tree, and
``abacus_amd/csrc/host/moe_host.cpp`` with g++ (OpenMP) into
``abacus_amd/lib/libabacus_moe_host.so``.
Run ``python -m abacus_amd.build`` (or ``__graft_entry__.build()``).
"""

from __future__ import annotations

import concurrent.futures
import os
import pathlib
import shutil
import subprocess
import sys

PKG = pathlib.Path(__file__).resolve().parent
INCLUDE = PKG.parent / "include"
CSRC = PKG / "csrc"
LIB_DIR = PKG / "lib"
LIB_NAME = "libabacus_moe.so"
HOST_LIB_NAME = "libabacus_moe_host.so"
# portable x86-64 code (no -march=native): the library is built here and runs on other hosts
HOST_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-fopenmp", "-shared", "-Wall", "-Wno-unused-parameter"]
ARCH = "gfx950"

# -packed-fp32-ops: never emit v_pk_{add,mul,fma}_f32 (see DESIGN notes on
# packed fp32); hipcc's host pass warns that it does not know the feature.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
    f"-I{INCLUDE}",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build libabacus_moe.so")
    return path


# Per-file additions.  attention.hip: MFMA results in VGPRs, not AGPRs -- its
# score and output accumulators are read and rescaled by VALU code every tile,
# and accumulators in AGPRs cost a move per element each way.
FILE_FLAGS = {"attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _compile(src: pathlib.Path, obj: pathlib.Path) -> None:
    cmd = [hipcc(), *HIPCC_FLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stdout}\n{res.stderr}")


def build_host(verbose: bool = True) -> pathlib.Path:
    """Compile the host C++ build of the C ABI (CPU tensors)."""
    cxx = shutil.which("g++") or shutil.which("c++")
    if cxx is None:
        raise RuntimeError("g++ not found; it builds libabacus_moe_host.so")
    LIB_DIR.mkdir(exist_ok=True)
    out = LIB_DIR / HOST_LIB_NAME
    tmp = LIB_DIR / (HOST_LIB_NAME + ".tmp")
    cmd = [cxx, *HOST_FLAGS, f"-I{INCLUDE}", str(CSRC / "host" / "moe_host.cpp"), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"g++ failed for moe_host.cpp:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}", file=sys.stderr)
    return out


def build(verbose: bool = True) -> pathlib.Path:
    """Compile all HIP sources for gfx950 and link the shared library, then the host library."""
    obj_dir = PKG / "_build"
    obj_dir.mkdir(exist_ok=True)
    LIB_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    objs = [obj_dir / (s.stem + ".o") for s in sources]
    jobs = min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        futures = [pool.submit(_compile, s, o) for s, o in zip(sources, objs)]
        for f in futures:
            f.result()
    out = LIB_DIR / LIB_NAME
    tmp = LIB_DIR / (LIB_NAME + ".tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}", file=sys.stderr)
    build_host(verbose)
    return out


if __name__ == "__main__":
    build()
