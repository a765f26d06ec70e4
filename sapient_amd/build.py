"""Build the gfx950 shared library ``sapient_amd/libsapient_hip.so``.

Each ``csrc/*.hip`` / ``csrc/*.cpp`` kernel translation unit and the C++
host layer (``host/*.cpp``) is compiled by hipcc (in parallel) into
``sapient_amd/_build/`` and linked into one shared library that exports the C
ABI declared in ``include/sapient_hip.h`` and the C++ API of
``include/sapient_hip_backend.hpp``.

Usage: ``python -m sapient_amd.build`` (or ``__graft_entry__.build()``).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libsapient_hip.so"

ARCH = "gfx950"

# Numerics flags are part of the parity contract:
#  -ffp-contract=off      no a*b+c fusion: products and sums round as in the reference
#  correctly-rounded f32 divide/sqrt, f32 denormals kept (both HIP defaults, stated)
#  -packed-fp32-ops off   no v_pk_{add,mul,fma}_f32 generation
#  -fma-mix/-mad-mix off  no v_fma_mix*/v_mad_mix*: the backend folds f32 products
#                         into these f16-result ops, which round differently from
#                         "round to f32, then to f16" and give +0 for -0 products
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Xclang", "-target-feature", "-Xclang", "-fma-mix-insts",
    "-Xclang", "-target-feature", "-Xclang", "-mad-mix-insts",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (expected /opt/rocm/bin/hipcc)")


def sources() -> list[Path]:
    return sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")) + list((PKG / "host").glob("*.cpp")))


def _compile(src: Path) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, f"-I{ROOT / 'include'}", f"-I{CSRC}", "-c", str(src), "-o", str(obj)]
    if src.suffix == ".cpp":
        cmd[1:1] = ["-x", "hip"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stderr}")
    return obj


def build(verbose: bool = True) -> Path:
    """Compile every translation unit for gfx950 and link the shared library."""
    BUILD.mkdir(exist_ok=True)
    srcs = sources()
    workers = max(1, min(len(srcs), os.cpu_count() or 1, 8))
    with cf.ThreadPoolExecutor(workers) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp),
           "-Wl,-rpath,/opt/rocm/lib"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB.relative_to(ROOT)} from {len(srcs)} sources")
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
