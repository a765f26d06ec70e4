"""The RoPE kernels evaluate sin and cos with sapient_amd/csrc/glibc_sincosf.h,
a restatement of glibc's sinf / cosf algorithm. This CPU test compiles that very
header for the host (tests/native/check_glibc_sincosf.cpp) and compares it with
the host libm's sinf, cosf and sincosf over all 2^32 f32 inputs. Zero
mismatches are required."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
NATIVE = ROOT / "tests" / "native"


@pytest.fixture(scope="module")
def harness():
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    out = NATIVE / "_build" / "check_glibc_sincosf"
    out.parent.mkdir(exist_ok=True)
    subprocess.run([gxx, "-O2", "-std=c++17", "-ffp-contract=off", "-fno-fast-math", "-D__HIP_PLATFORM_AMD__",
                    "-I/opt/rocm/include", f"-I{ROOT / 'sapient_amd' / 'csrc'}", f"-I{ROOT / 'include'}",
                    str(NATIVE / "check_glibc_sincosf.cpp"), "-o", str(out), "-lpthread", "-lm"], check=True)
    return out


def test_sinf_cosf_bit_exact_over_all_f32(harness):
    res = subprocess.run([str(harness), "8"], capture_output=True, text=True, timeout=600)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "sinf mismatches 0" in res.stdout and "cosf mismatches 0" in res.stdout
