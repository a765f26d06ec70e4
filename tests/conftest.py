"""Shared pytest set-up: import paths, the `gpu` marker, device and oracle fixtures."""
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: runs HIP kernels; needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def orc():
    """The CPU oracle (built on first use)."""
    import oracle
    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def dev():
    """cuda:0 with the HIP library loaded; fails (never skips) without a GPU."""
    import torch
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    import sapient_amd
    if not sapient_amd.LIB_PATH.exists():
        from sapient_amd import build
        build.build()
    sapient_amd.lib()
    return torch.device("cuda:0")
