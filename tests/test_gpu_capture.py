"""HIP graph capture of the op set: the GELU tables' one-time build refuses to run under capture (it
waits for its kernels), and once built, captured GELU launches replay correctly.

Runs in a child process so that the library's one-time set-up has not yet happened there.
"""
import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]

CHILD = r'''
import sys
sys.path.insert(0, sys.argv[1])
import torch
import sapient_amd.ops as ops
from sapient_amd._lib import ESTATE, SapientHipError
dev = torch.device("cuda:0")
g = torch.Generator(device=dev).manual_seed(3)
for dt in (torch.float16, torch.bfloat16):
    x = (torch.randn(1 << 20, generator=g, device=dev) * 2).to(dt)
    out = torch.empty_like(x)
    status = None
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        try:
            ops.gelu_tanh(x, out=out)
        except SapientHipError as e:
            status = e.status
    print("lazy set-up under capture:", status, flush=True)
    assert status == ESTATE, status
    del graph
ops.init(dev)
for fn in (ops.gelu_tanh, ops.gelu_erf):
    for dt in (torch.float16, torch.bfloat16):
        x = (torch.randn(1 << 20, generator=g, device=dev) * 2).to(dt)
        want = fn(x)
        out = torch.empty_like(x)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            fn(x, out=out)
        for r in range(3):
            out.zero_()
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out.view(torch.int16), want.view(torch.int16)), (fn.__name__, dt, r)
        print("replayed", fn.__name__, dt, flush=True)
print("capture: ok", flush=True)
'''


def test_gelu_table_build_refused_under_capture_and_captured_gelu_replays():
    print("case capture: lazy GELU set-up under capture, then captured GELU replays", flush=True)
    res = subprocess.run([sys.executable, "-c", CHILD, str(ROOT)], capture_output=True, text=True, timeout=300)
    print(res.stdout[-2000:], res.stderr[-2000:], flush=True)
    assert res.returncode == 0 and "capture: ok" in res.stdout
