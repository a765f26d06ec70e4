"""GPU parity: RoPE with the angles read from cos / sin tables (sph_rope_cached).

Reference: crates/sapient-backends/cpu/src/kernels/rope.rs:18-62 (apply_rope),
:83-136 (apply_rope_partial_scaled) and :140-153 (rope_cos_sin_cache, the
table layout). The trait path's LlmBackend::apply_rope_positions
(crates/sapient-models/src/forward/backend.rs:84) holds its positions on the
host; the library's host function sph_rope_table evaluates their angles with
the host libm, as the reference does, and the kernel only reads them.

Bar: bit-exact with the oracle, as sph_rope.
"""
import numpy as np
import pytest
import torch

from helpers import narrow_bits, to_np, widen

import sapient_amd.ops as ops

pytestmark = pytest.mark.gpu
IDS = lambda d: str(d).split(".")[-1]


def _gen(shape, seed, dev, dtype=torch.float32):
    g = torch.Generator(device=dev).manual_seed(seed)
    return torch.randn(shape, generator=g, device=dev).to(dtype)


def _check(out: torch.Tensor, ref32: np.ndarray, orc, what):
    if out.dtype == torch.float32:
        got = to_np(out).reshape(-1).view(np.uint32)
        want = np.ascontiguousarray(ref32, np.float32).reshape(-1).view(np.uint32)
    else:
        got = to_np(out).reshape(-1)
        want = narrow_bits(np.ascontiguousarray(ref32, np.float32), out.dtype, orc).reshape(-1)
    bad = np.flatnonzero(got != want)
    if bad.size:
        i = bad[:5]
        raise AssertionError(f"{what}: {bad.size} of {got.size} elements differ; first {i.tolist()}: "
                             f"got {got[i]} want {want[i]}")


def _run(dev, orc, dtype, B, Hq, Hk, S, D, rd, base, positions, interleaved, mode, pos_scale=1.0, seed=0):
    """mode "call": tables for exactly this call's positions, no device positions (the trait path);
    mode "cache": one table over positions 0 .. max(positions) and device positions indexing it."""
    q = _gen((B, Hq, S, D), 100 + seed, dev, dtype)
    k = _gen((B, Hk, S, D), 200 + seed, dev, dtype) if Hk else None
    q32 = widen(q, orc).reshape(B, Hq, S, D)
    k32 = widen(k, orc).reshape(B, Hk, S, D) if Hk else None
    if mode == "call":
        ops.rope_host_positions_(q, k, positions, base, rotary_dim=rd, pos_scale=pos_scale, interleaved=interleaved)
    else:
        cs, sn = ops.rope_table(None, rd, base, pos_scale, n=max(positions) + 1)
        pos = torch.tensor(positions, dtype=torch.int32, device=dev)
        ops.rope_cached_(q, k, torch.from_numpy(cs).to(dev), torch.from_numpy(sn).to(dev), pos, rd, interleaved)
    torch.cuda.synchronize()
    what = f"rope_cached {mode} {'il' if interleaved else 'neox'} {dtype} B{B} Hq{Hq} Hk{Hk} S{S} D{D} rd{rd}"
    _check(q, orc.apply_rope_partial_scaled(q32, positions, base, rd, pos_scale, interleaved), orc, what + " q")
    if Hk:
        _check(k, orc.apply_rope_partial_scaled(k32, positions, base, rd, pos_scale, interleaved), orc, what + " k")


@pytest.mark.parametrize("mode", ["call", "cache"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16], ids=IDS)
@pytest.mark.parametrize("interleaved", [False, True], ids=["neox", "interleaved"])
@pytest.mark.parametrize("B,Hq,Hk,S,D,rd", [
    (1, 14, 2, 1, 64, 64),       # Qwen2.5-0.5B decode (T = 1)
    (1, 14, 2, 512, 64, 64),     # Qwen2.5-0.5B prefill (T = 512)
    (2, 4, 2, 9, 128, 128),
    (1, 3, 0, 5, 80, 32),        # Phi partial rotary
    (1, 2, 1, 3, 6, 6),          # odd half: one pair per thread
    (1, 2, 2, 4, 12, 8),
    (1, 3, 2, 37, 16, 12),
    (1, 5, 1, 300, 40, 40),
])
def test_rope_cached_shapes(dev, orc, mode, dtype, interleaved, B, Hq, Hk, S, D, rd):
    positions = [int(p) for p in np.random.default_rng(S).integers(0, 8192, S)] if S > 1 else [4095]
    base = 1e6 if D == 64 else 5e5
    print(f"case rope_cached {mode} {dtype} il={interleaved} {B},{Hq},{Hk},{S},{D},{rd}", flush=True)
    _run(dev, orc, dtype, B, Hq, Hk, S, D, rd, base, positions, interleaved, mode)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=IDS)
@pytest.mark.parametrize("interleaved", [False, True], ids=["neox", "interleaved"])
def test_rope_cached_llama3_8b_full(dev, orc, dtype, interleaved):
    """Q 32 heads + K 8 heads, T = 8192 contiguous positions, head_dim 128, theta 5e5, from a cached table."""
    print(f"case rope_cached full {dtype} il={interleaved}", flush=True)
    _run(dev, orc, dtype, 1, 32, 8, 8192, 128, 128, 5e5, list(range(8192)), interleaved, "cache", seed=7)


@pytest.mark.parametrize("mode", ["call", "cache"])
def test_rope_cached_linear_position_scale(dev, orc, mode):
    """rope.rs:123-124: effective position pos / pos_scale, folded into the table."""
    print(f"case rope_cached pos_scale 8 {mode}", flush=True)
    _run(dev, orc, torch.float32, 1, 4, 2, 33, 128, 128, 1e6, list(range(100, 133)), False, mode, pos_scale=8.0)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=IDS)
@pytest.mark.parametrize("offset", [1, 2])
def test_rope_cached_unaligned_rows(dev, orc, dtype, offset):
    """q and k starting `offset` elements into their buffers take the narrower access paths."""
    B, Hq, Hk, S, D = 1, 5, 3, 11, 32
    g = torch.Generator(device=dev).manual_seed(offset)
    bq = torch.randn(offset + B * Hq * S * D, generator=g, device=dev).to(dtype)
    bk = torch.randn(offset + B * Hk * S * D, generator=g, device=dev).to(dtype)
    q, k = bq[offset:].view(B, Hq, S, D), bk[offset:].view(B, Hk, S, D)
    q32, k32 = widen(q.contiguous(), orc).reshape(B, Hq, S, D), widen(k.contiguous(), orc).reshape(B, Hk, S, D)
    positions = [int(p) for p in np.random.default_rng(offset).integers(0, 8192, S)]
    print(f"case rope_cached unaligned {dtype} offset {offset}", flush=True)
    ops.rope_host_positions_(q, k, positions, 5e5)
    torch.cuda.synchronize()
    _check(q, orc.apply_rope_partial_scaled(q32, positions, 5e5, D, 1.0, False), orc, "q")
    _check(k, orc.apply_rope_partial_scaled(k32, positions, 5e5, D, 1.0, False), orc, "k")


def test_rope_cached_positions_outside_the_table(dev, orc):
    """A position outside [0, table_rows) leaves its token unchanged and raises the flag; the others rotate."""
    B, Hq, Hk, S, D = 1, 3, 1, 6, 64
    positions = [5, -1, 7, 8, 100, 2]  # table rows 0 .. 7: tokens 1, 3 and 4 are outside
    q = _gen((B, Hq, S, D), 11, dev)
    k = _gen((B, Hk, S, D), 12, dev)
    q0, k0 = to_np(q).copy(), to_np(k).copy()
    cs, sn = ops.rope_table(None, D, 1e4, n=8)
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    print("case rope_cached bad positions", flush=True)
    ops.rope_cached_(q, k, torch.from_numpy(cs).to(dev), torch.from_numpy(sn).to(dev),
                     torch.tensor(positions, dtype=torch.int32, device=dev), bad_pos_flag=flag)
    torch.cuda.synchronize()
    assert int(flag.item()) == 1
    for s, p in enumerate(positions):
        for x, x0 in ((q, q0), (k, k0)):
            got = to_np(x)[:, :, s]
            if 0 <= p < 8:
                ref = orc.apply_rope_partial_scaled(x0[:, :, s:s + 1], [p], 1e4, D)
                assert np.array_equal(got.view(np.uint32), ref[:, :, 0].view(np.uint32)), f"token {s}"
            else:
                assert np.array_equal(got.view(np.uint32), x0[:, :, s].view(np.uint32)), f"token {s} changed"
    flag.zero_()
    ops.rope_cached_(q, k, torch.from_numpy(cs).to(dev), torch.from_numpy(sn).to(dev),
                     torch.tensor([0, 1, 2, 3, 4, 5], dtype=torch.int32, device=dev), bad_pos_flag=flag)
    torch.cuda.synchronize()
    assert int(flag.item()) == 0


def test_rope_cached_rejects_bad_arguments(dev):
    from sapient_amd._lib import EINVAL, ERANGE, lib
    q = torch.zeros(1, 2, 4, 8, device=dev)
    t = torch.zeros(4, 4, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    L = lib()
    # no tables; tables of 3 rows for 4 tokens without positions; odd head_dim; rotary_dim > head_dim; bad layout
    assert L.sph_rope_cached(q.data_ptr(), 2, None, 0, 0, 0, None, t.data_ptr(), 4, None, 1, 4, 8, 8, None, s) == EINVAL
    assert L.sph_rope_cached(q.data_ptr(), 2, None, 0, 0, 0, t.data_ptr(), t.data_ptr(), 3, None, 1, 4, 8, 8, None,
                             s) == ERANGE
    assert L.sph_rope_cached(q.data_ptr(), 2, None, 0, 0, 0, t.data_ptr(), t.data_ptr(), 4, None, 1, 4, 7, 6, None,
                             s) == EINVAL
    assert L.sph_rope_cached(q.data_ptr(), 2, None, 0, 0, 0, t.data_ptr(), t.data_ptr(), 4, None, 1, 4, 8, 10, None,
                             s) == EINVAL
    assert L.sph_rope_cached(q.data_ptr(), 2, None, 0, 0, 2, t.data_ptr(), t.data_ptr(), 4, None, 1, 4, 8, 8, None,
                             s) == EINVAL
    assert L.sph_rope_cached(q.data_ptr(), 2, None, 0, 0, 0, t.data_ptr() + 2, t.data_ptr(), 4, None, 1, 4, 8, 8,
                             None, s) == EINVAL
    torch.cuda.synchronize()
    assert not q.any()
