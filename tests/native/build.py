"""Builds the native test programs of tests/native/ into tests/native/_build/:

- test_hip_llm_backend: GPU tests of the C++ LlmBackend mirror, linked against the
  in-tree libsapient_hip.so (rpath relative to the binary, so the tree can move);
- test_tensor_host: the mirror's Tensor and byte storage, no GPU needed;
- bench_host_tensor: the mirror's host-tensor rate, run by bench.py;
- check_glibc_tanhf, check_glibc_expf, check_glibc_sincosf: the host-side
  exhaustive checks of glibc_tanhf.h, glibc_expf.h and glibc_sincosf.h.
"""
import shutil
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
OUT = HERE / "_build"


def build() -> None:
    gxx = shutil.which("g++") or "g++"
    OUT.mkdir(exist_ok=True)
    subprocess.run([gxx, "-std=c++17", "-O1", "-Wall", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
                    f"-I{ROOT / 'include'}", str(HERE / "test_hip_llm_backend.cpp"),
                    "-o", str(OUT / "test_hip_llm_backend"), f"-L{ROOT / 'sapient_amd'}", "-lsapient_hip",
                    "-L/opt/rocm/lib", "-lamdhip64",
                    "-Wl,-rpath,$ORIGIN/../../../sapient_amd", "-Wl,-rpath,/opt/rocm/lib"], check=True)
    for prog in ("bench_host_tensor", "test_tensor_host"):
        subprocess.run([gxx, "-std=c++17", "-O2", "-Wall", f"-I{ROOT / 'include'}", str(HERE / f"{prog}.cpp"),
                        "-o", str(OUT / prog), f"-L{ROOT / 'sapient_amd'}", "-lsapient_hip",
                        "-Wl,-rpath,$ORIGIN/../../../sapient_amd", "-Wl,-rpath,/opt/rocm/lib"], check=True)
    for check in ("check_glibc_tanhf", "check_glibc_expf", "check_glibc_sincosf"):
        subprocess.run([gxx, "-O2", "-std=c++17", "-ffp-contract=off", "-fno-fast-math", "-D__HIP_PLATFORM_AMD__",
                        "-I/opt/rocm/include", f"-I{ROOT / 'sapient_amd' / 'csrc'}", f"-I{ROOT / 'include'}",
                        str(HERE / f"{check}.cpp"), "-o", str(OUT / check), "-lpthread", "-lm"], check=True)


if __name__ == "__main__":
    build()
