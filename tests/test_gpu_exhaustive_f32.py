"""GPU parity over every f32 input: the f32 SiLU, GELU-tanh and erf-GELU kernels
against the oracle, all 2^32 bit patterns each, and the device's f32 -> f16 /
bf16 narrowing (through kv_append) against the oracle's half conversion.

Reference: crates/sapient-backends/cpu/src/kernels/elementwise.rs:141-143 (silu),
:120-127 (gelu, tanh form), :135-138 with erf_approx :163-174 (gelu_erf).

The device evaluates glibc's expf and tanhf/expm1f as restated in
sapient_amd/csrc/glibc_expf.h and glibc_tanhf.h. Those headers are checked
against the host libm over every input when compiled for the host
(tests/test_glibc_*_restatement.py); this test checks the device binary itself,
every input through the product kernels, against the oracle (glibc libm on this
host). Bar: bit-exact; NaN where the oracle gives NaN (payloads are each
platform's own).

The oracle runs on the host's cores in parallel (its C loops release the GIL
through ctypes), chunk by chunk, beside the GPU.
"""
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest
import torch

import sapient_amd.ops as ops

pytestmark = pytest.mark.gpu

CHUNK = 1 << 27  # bit patterns per chunk; divides 2^31, so no chunk crosses the sign bit
OPS = {
    "silu": (ops.silu, "sor_silu"),
    "gelu_tanh": (ops.gelu_tanh, "sor_gelu"),
    "gelu_erf": (ops.gelu_erf, "sor_gelu_erf"),
}


def _oracle_chunk(fn, x: np.ndarray, pool, nthreads: int) -> np.ndarray:
    out = np.empty_like(x)
    step = (x.size + nthreads - 1) // nthreads
    futs = []
    for i in range(0, x.size, step):
        xs, os_ = x[i:i + step], out[i:i + step]
        futs.append(pool.submit(fn, xs.ctypes.data, os_.ctypes.data, xs.size))
    for f in futs:
        f.result()
    return out


@pytest.mark.parametrize("name", list(OPS))
def test_f32_activation_every_input(dev, orc, name):
    op, sym = OPS[name]
    fn = getattr(orc.lib(), sym)
    nthreads = max(1, min(16, os.cpu_count() or 1))
    ops.init(dev)
    bad = nan_bad = 0
    first = None
    with ThreadPoolExecutor(nthreads) as pool:
        for c in range((1 << 32) // CHUNK):
            start = c * CHUNK if c * CHUNK < (1 << 31) else c * CHUNK - (1 << 32)  # as int32
            xb = torch.arange(start, start + CHUNK, dtype=torch.int32, device=dev)
            got = op(xb.view(torch.float32)).view(torch.int32)
            ref_np = _oracle_chunk(fn, np.arange(start, start + CHUNK, dtype=np.int32).view(np.float32), pool,
                                   nthreads)
            ref = torch.from_numpy(ref_np.view(np.int32)).to(dev)
            nan_g = (got & 0x7FFFFFFF) > 0x7F800000
            nan_r = (ref & 0x7FFFFFFF) > 0x7F800000
            nan_bad += int((nan_g != nan_r).sum())
            diff = (got != ref) & ~nan_r
            nd = int(diff.sum())
            if nd and first is None:
                i = int(torch.nonzero(diff)[0])
                first = (hex((start + i) & 0xFFFFFFFF), hex(int(got[i]) & 0xFFFFFFFF), hex(int(ref[i]) & 0xFFFFFFFF))
            bad += nd
            if c % 8 == 7:
                print(f"case {name} f32 every input: {c + 1} of 32 chunks, mismatches {bad}, NaN mismatches {nan_bad}",
                      flush=True)
    assert bad == 0 and nan_bad == 0, f"{name}: {bad} outputs differ, {nan_bad} NaN mismatches; first (x, got, want) {first}"


@pytest.mark.parametrize("half", ["f16", "bf16"])
def test_f32_to_half_every_input(dev, orc, half):
    """Every kernel that stores f16 / bf16 words narrows pairs with the same device
    helpers, narrow2_f16 (v_cvt_pk_f16_f32) and narrow2_bf16 (v_cvt_pk_bf16_f32).
    kv_append from an f32 source into a half cache at head_dim 128 (8-element
    items) is that packed narrowing alone, so this sweep pins the packed
    conversion over every f32 input; the oracle's is half's from_f32 (round bit
    and sticky bits, NaN quieted with 0x40 for bf16). Bar: bit-exact, NaN included."""
    tdt = torch.float16 if half == "f16" else torch.bfloat16
    fn = getattr(orc.lib(), "sor_f32_to_f16_n" if half == "f16" else "sor_f32_to_bf16_n")
    nthreads = max(1, min(16, os.cpu_count() or 1))
    ops.init(dev)
    hd = 128
    cache = torch.empty((1, CHUNK // hd, hd), dtype=tdt, device=dev)
    bad = 0
    first = None
    with ThreadPoolExecutor(nthreads) as pool:
        for c in range((1 << 32) // CHUNK):
            start = c * CHUNK if c * CHUNK < (1 << 31) else c * CHUNK - (1 << 32)
            xb = torch.arange(start, start + CHUNK, dtype=torch.int32, device=dev)
            ops.kv_append(xb.view(torch.float32).view(1, CHUNK // hd, hd), cache, 0)
            got = cache.view(torch.int16).flatten()
            x_np = np.arange(start, start + CHUNK, dtype=np.int32).view(np.float32)
            ref_np = np.empty(CHUNK, dtype=np.uint16)
            step = (CHUNK + nthreads - 1) // nthreads
            futs = [pool.submit(fn, x_np[i:i + step].ctypes.data, ref_np[i:i + step].ctypes.data, x_np[i:i + step].size)
                    for i in range(0, CHUNK, step)]
            for f in futs:
                f.result()
            ref = torch.from_numpy(ref_np.view(np.int16)).to(dev)
            diff = got != ref
            nd = int(diff.sum())
            if nd and first is None:
                i = int(torch.nonzero(diff)[0])
                first = (hex((start + i) & 0xFFFFFFFF), hex(int(got[i]) & 0xFFFF), hex(int(ref[i]) & 0xFFFF))
            bad += nd
            if c % 8 == 7:
                print(f"case f32 -> {half} every input: {c + 1} of 32 chunks, mismatches {bad}", flush=True)
    assert bad == 0, f"f32 -> {half}: {bad} outputs differ; first (x, got, want) {first}"
