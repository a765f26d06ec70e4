"""CPU: the C++ mirror's Tensor and byte storage (include/sapient_hip_backend.hpp) pass their
host-only test program (tests/native/test_tensor_host.cpp) — construction checks, shared bytes with
copy on write, byte counts of the block formats, and storage growth — with no GPU present."""
import subprocess
from pathlib import Path

NATIVE = Path(__file__).resolve().parent / "native"


def test_tensor_host_program():
    exe = NATIVE / "_build" / "test_tensor_host"
    if not exe.exists():
        import sapient_amd
        if not sapient_amd.LIB_PATH.exists():  # the program links the library
            from sapient_amd import build
            build.build()
        import importlib.util
        spec = importlib.util.spec_from_file_location("native_build", NATIVE / "build.py")
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        mod.build()
    res = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert res.returncode == 0, res.stdout + res.stderr
    assert res.stdout.strip().endswith("0 failed"), res.stdout
