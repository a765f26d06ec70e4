"""The erf-GELU kernels evaluate exp with sapient_amd/csrc/glibc_expf.h, a
restatement of glibc's expf algorithm. This CPU test compiles that very header
for the host (tests/native/check_glibc_expf.cpp) and compares it — and the SiLU
and whole erf-GELU expressions in the reference's operation order — with the
host libm over all 2^32 f32 inputs. Zero mismatches are required."""
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
    out = NATIVE / "_build" / "check_glibc_expf"
    out.parent.mkdir(exist_ok=True)
    subprocess.run([gxx, "-O2", "-std=c++17", "-ffp-contract=off", "-fno-fast-math", "-D__HIP_PLATFORM_AMD__",
                    "-I/opt/rocm/include", f"-I{ROOT / 'sapient_amd' / 'csrc'}", f"-I{ROOT / 'include'}",
                    str(NATIVE / "check_glibc_expf.cpp"), "-o", str(out), "-lpthread", "-lm"], check=True)
    return out


def test_expf_silu_and_gelu_erf_bit_exact_over_all_f32(harness):
    res = subprocess.run([str(harness), "8"], capture_output=True, text=True, timeout=600)
    assert res.returncode == 0, res.stdout + res.stderr
    for name in ("expf", "expf_nonpos", "silu", "gelu_erf"):
        assert f"{name} mismatches 0" in res.stdout
