"""GPU parity over every (gate, up) pair of the half-precision SwiGLU: all
2^32 combinations of the 65536 gate and 65536 up bit patterns, f16 and bf16.

Reference: crates/sapient-backends/cpu/src/kernels/elementwise.rs:141-143
(silu: g / (1 + expf(-g))) then :67-69 (mul), in f32 from the widened halves;
the half output is that f32 product rounded once, to nearest-even.

The half kernels evaluate a fast SiLU and keep its result only where a
certificate shows that every f32 near it rounds to the same half value as the
reference's exact product; this test checks the claim on every input pair
instead of relying on the fast SiLU's measured error bound.

Expected values, on the host: silu(gate) for every gate pattern from the
oracle (glibc's expf, the reference's op order), the IEEE f32 product with the
widened up value (numpy), and the oracle's round-to-nearest-even narrowing,
run on the host's cores in parallel chunk by chunk. A random sample of pairs
is checked against the oracle's whole SwiGLU first, so the composition is the
oracle's. Bar: bit-exact; NaN where the expected value is NaN (payloads are
each platform's own).
"""
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest
import torch

from helpers import to_np

import sapient_amd.ops as ops

pytestmark = pytest.mark.gpu

GATES_PER_CHUNK = 4096  # 2^28 pairs per launch


def _nan16(b: np.ndarray, half: str) -> np.ndarray:
    if half == "f16":
        return ((b & 0x7C00) == 0x7C00) & ((b & 0x3FF) != 0)
    return ((b & 0x7F80) == 0x7F80) & ((b & 0x7F) != 0)


@pytest.mark.parametrize("half", ["f16", "bf16"])
def test_half_swiglu_every_gate_up_pair(dev, orc, half):
    tdt = torch.float16 if half == "f16" else torch.bfloat16
    widen = orc.f16_bits_to_f32 if half == "f16" else orc.bf16_bits_to_f32
    narrow = orc.f32_to_f16_bits if half == "f16" else orc.f32_to_bf16_bits
    narrow_n = getattr(orc.lib(), "sor_f32_to_f16_n" if half == "f16" else "sor_f32_to_bf16_n")
    pats = np.arange(65536, dtype=np.uint16)
    s = orc.silu(widen(pats))  # the oracle's silu of every gate pattern
    u = widen(pats)            # every up value, widened exactly

    # The composition below equals the oracle's whole SwiGLU on a sample of pairs.
    rng = np.random.default_rng(5)
    gs, us = rng.integers(0, 65536, 8192), rng.integers(0, 65536, 8192)
    want = narrow(orc.swiglu(widen(gs.astype(np.uint16)), u[us]))
    comp = narrow(s[gs] * u[us])
    assert np.array_equal(_nan16(comp, half), _nan16(want, half))
    assert np.array_equal(comp[~_nan16(want, half)], want[~_nan16(want, half)])

    nthreads = max(1, min(16, os.cpu_count() or 1))
    up = torch.from_numpy(pats.view(np.int16)).to(dev).view(tdt)[None, :].expand(GATES_PER_CHUNK, 65536).contiguous()
    bad = nan_bad = 0
    first = None
    n = GATES_PER_CHUNK * 65536
    ref = np.empty(n, np.uint16)
    with ThreadPoolExecutor(nthreads) as pool:
        for c in range(65536 // GATES_PER_CHUNK):
            g0 = c * GATES_PER_CHUNK
            gate = torch.from_numpy(pats[g0:g0 + GATES_PER_CHUNK].view(np.int16)).to(dev).view(tdt)
            gate = gate[:, None].expand(GATES_PER_CHUNK, 65536).contiguous()
            got = to_np(ops.swiglu(gate, up)).reshape(-1)
            prod = (s[g0:g0 + GATES_PER_CHUNK, None] * u[None, :]).reshape(-1)
            step = (n + nthreads - 1) // nthreads
            futs = [pool.submit(narrow_n, prod[i:i + step].ctypes.data, ref[i:i + step].ctypes.data,
                                prod[i:i + step].size) for i in range(0, n, step)]
            for f in futs:
                f.result()
            nan_g, nan_r = _nan16(got, half), _nan16(ref, half)
            nan_bad += int(np.count_nonzero(nan_g != nan_r))
            diff = (got != ref) & ~nan_r
            nd = int(np.count_nonzero(diff))
            if nd and first is None:
                i = int(np.flatnonzero(diff)[0])
                first = (hex(g0 + i // 65536), hex(i % 65536), hex(int(got[i])), hex(int(ref[i])))
            bad += nd
            if c % 4 == 3:
                print(f"case {half} swiglu every (gate, up): {c + 1} of 16 chunks, mismatches {bad}, "
                      f"NaN mismatches {nan_bad}", flush=True)
            del gate, got, prod, nan_g, nan_r, diff
    assert bad == 0 and nan_bad == 0, \
        f"{half} swiglu: {bad} outputs differ, {nan_bad} NaN mismatches; first (gate, up, got, want) {first}"
