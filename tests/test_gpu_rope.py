"""GPU parity: rotary position embedding (NEOX and interleaved), in place.

Reference: crates/sapient-backends/cpu/src/kernels/rope.rs:18-62 (apply_rope),
:83-136 (apply_rope_partial_scaled); interleaved pairs per the GGUF q/k row
permutation (crates/sapient-models/src/gguf_weights.rs:111-115).

Bar: bit-exact. The denominators are the host libm's powf (as the reference
calls it), sin and cos are glibc's sinf / cosf restated (exhaustively equal to
the host libm, tests/test_glibc_sincosf_restatement.py), and the rotation
rounds each product before the add or subtract, as the oracle does. f32
outputs equal the oracle's bits; half outputs equal the oracle's f32 result
rounded to nearest-even.
"""
import numpy as np
import pytest
import torch

from helpers import narrow_bits, to_np, widen
from refvec import WgpuLcg

import sapient_amd.ops as ops

pytestmark = pytest.mark.gpu


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


def _run(dev, orc, dtype, B, Hq, Hk, S, D, rd, base, positions, interleaved, pos_scale=1.0, seed=0):
    q = _gen((B, Hq, S, D), 100 + seed, dev, dtype)
    k = _gen((B, Hk, S, D), 200 + seed, dev, dtype) if Hk else None
    q32 = widen(q, orc).reshape(B, Hq, S, D)
    k32 = widen(k, orc).reshape(B, Hk, S, D) if Hk else None
    pos = torch.tensor(positions, dtype=torch.int32, device=dev)
    ops.rope_(q, k, pos, base, rotary_dim=rd, pos_scale=pos_scale, interleaved=interleaved)
    torch.cuda.synchronize()
    what = f"rope {'il' if interleaved else 'neox'} {dtype} B{B} Hq{Hq} Hk{Hk} S{S} D{D} rd{rd}"
    ref_q = orc.apply_rope_partial_scaled(q32, positions, base, rd, pos_scale, interleaved)
    _check(q, ref_q, orc, what + " q")
    if Hk:
        ref_k = orc.apply_rope_partial_scaled(k32, positions, base, rd, pos_scale, interleaved)
        _check(k, ref_k, orc, what + " k")


@pytest.mark.parametrize("H,S,D,rd", [(4, 7, 80, 32), (3, 5, 64, 64)])
def test_rope_matches_wgpu_test_vectors(dev, orc, H, S, D, rd):
    """resident.rs:152-187: lcg 0x9E3779B9 data, positions s + 11, base 1e4."""
    nxt = WgpuLcg()
    data = nxt.take(H * S * D).reshape(1, H, S, D)
    positions = [s + 11 for s in range(S)]
    x = torch.from_numpy(data.copy()).to(dev)
    print(f"case rope wgpu-vectors {H},{S},{D},{rd}", flush=True)
    ops.rope_(x, None, torch.tensor(positions, dtype=torch.int32, device=dev), 1e4, rotary_dim=rd)
    ref = orc.apply_rope_partial_scaled(data, positions, 1e4, rd)
    _check(x, ref, orc, "rope wgpu vectors")
    assert np.abs(to_np(x) - ref).max() < 1e-4  # the reference test's own bound


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16], ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("interleaved", [False, True], ids=["neox", "interleaved"])
@pytest.mark.parametrize("B,Hq,Hk,S,D,rd", [
    (1, 14, 2, 1, 64, 64),       # Qwen2.5-0.5B decode (T = 1)
    (1, 14, 2, 512, 64, 64),     # Qwen2.5-0.5B prefill (T = 512)
    (2, 4, 2, 9, 128, 128),
    (1, 3, 0, 5, 80, 32),        # Phi partial rotary
    (1, 2, 1, 3, 6, 6),          # odd half: scalar path
    (1, 2, 2, 4, 12, 8),
    (1, 3, 2, 37, 16, 12),       # half = 6: interleaved one run per thread (no split), NEOX with 2-pair runs
    (1, 5, 1, 300, 40, 40),      # half = 20: more tokens than one block, split interleaved
])
def test_rope_shapes(dev, orc, dtype, interleaved, B, Hq, Hk, S, D, rd):
    positions = [int(p) for p in np.random.default_rng(S).integers(0, 8192, S)] if S > 1 else [4095]
    base = 1e6 if D == 64 else 5e5
    print(f"case rope {dtype} il={interleaved} {B},{Hq},{Hk},{S},{D},{rd}", flush=True)
    _run(dev, orc, dtype, B, Hq, Hk, S, D, rd, base, positions, interleaved)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16], ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("interleaved", [False, True], ids=["neox", "interleaved"])
@pytest.mark.parametrize("offset", [1, 2, 4])
def test_rope_unaligned_rows(dev, orc, dtype, interleaved, offset):
    """q and k starting `offset` elements into their buffers: narrower accesses than the 16-byte paths."""
    B, Hq, Hk, S, D = 1, 5, 3, 11, 32
    g = torch.Generator(device=dev).manual_seed(offset)
    bq = torch.randn(offset + B * Hq * S * D, generator=g, device=dev).to(dtype)
    bk = torch.randn(offset + B * Hk * S * D, generator=g, device=dev).to(dtype)
    q, k = bq[offset:].view(B, Hq, S, D), bk[offset:].view(B, Hk, S, D)
    q32, k32 = widen(q.contiguous(), orc).reshape(B, Hq, S, D), widen(k.contiguous(), orc).reshape(B, Hk, S, D)
    positions = [int(p) for p in np.random.default_rng(offset).integers(0, 8192, S)]
    print(f"case rope unaligned {dtype} il={interleaved} offset {offset}", flush=True)
    ops.rope_(q, k, torch.tensor(positions, dtype=torch.int32, device=dev), 5e5, interleaved=interleaved)
    torch.cuda.synchronize()
    what = f"rope unaligned {dtype} il={interleaved} offset {offset}"
    _check(q, orc.apply_rope_partial_scaled(q32, positions, 5e5, D, 1.0, interleaved), orc, what + " q")
    _check(k, orc.apply_rope_partial_scaled(k32, positions, 5e5, D, 1.0, interleaved), orc, what + " k")


def test_rope_linear_position_scale(dev, orc):
    """rope.rs:123-124: effective position pos / pos_scale (Gemma3 uses 8)."""
    _run(dev, orc, torch.float32, 1, 4, 2, 33, 128, 128, 1e6, list(range(100, 133)), False, pos_scale=8.0)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16], ids=["float32", "float16"])
@pytest.mark.parametrize("interleaved", [False, True], ids=["neox", "interleaved"])
def test_rope_llama3_8b_full(dev, orc, dtype, interleaved):
    """Q 32 heads + K 8 heads, T = 8192 contiguous positions, head_dim 128, theta 5e5."""
    print(f"case rope full {dtype} il={interleaved}", flush=True)
    _run(dev, orc, dtype, 1, 32, 8, 8192, 128, 128, 5e5, list(range(8192)), interleaved, seed=7)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=["float16", "bfloat16"])
@pytest.mark.parametrize("interleaved", [False, True], ids=["neox", "interleaved"])
def test_rope_head_groups_with_a_single_head_batch(dev, orc, dtype, interleaved):
    """32 + 4 heads x 8192 tokens: the half-type kernel splits the 36 heads into four groups of 9, so
    after the eight heads requested before the angle phase (four batches of two) a group ends with a
    batch holding one head. Bit-exact like every other shape."""
    print(f"case rope 9-head groups {dtype} il={interleaved}", flush=True)
    _run(dev, orc, dtype, 1, 32, 4, 8192, 128, 128, 5e5, list(range(8192)), interleaved, seed=9)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16], ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("interleaved", [False, True], ids=["neox", "interleaved"])
@pytest.mark.parametrize("pos_scale", [1.0, 7.5, 2.0 ** -7, 3.0e-5, 2.0 ** -20, 1e-30])
def test_rope_device_sin_cos_equal_glibc(dev, orc, pos_scale, interleaved, dtype):
    """A (1, 0) pair with head_dim 2 rotates to exactly (cos θ, sin θ), θ = (pos / pos_scale) / base⁰. Over 2^20
    positions in [0, 2^31) — random, plus the first 4096 — and pos_scales from 7.5 down to 1e-30, the angles span
    zero, both reduction ranges (below and above 120, every window of the 4/pi table) and overflow to inf: every
    output equals the oracle's glibc sinf / cosf bit for bit (NaN where θ is inf, on both sides; NaN payloads are
    the platforms' own)."""
    S = 1 << 20
    rng = np.random.default_rng(2024)
    pos = rng.integers(0, 2 ** 31 - 1, S, dtype=np.int64).astype(np.int32)
    pos[:4096] = np.arange(4096, dtype=np.int32)
    x = np.zeros((1, 1, S, 2), np.float32)
    x[..., 0] = 1.0
    t = torch.from_numpy(x).to(dev).to(dtype)  # 1 and 0 are exact in every type
    print(f"case rope sin/cos pos_scale {pos_scale} il={interleaved} {dtype}", flush=True)
    ops.rope_(t, None, torch.from_numpy(pos).to(dev), 1e4, pos_scale=pos_scale, interleaved=interleaved)
    ref = orc.apply_rope_partial_scaled(x, pos, 1e4, 2, pos_scale, interleaved).reshape(-1)
    nan = np.isnan(ref)
    if dtype == torch.float32:
        got = to_np(t).reshape(-1)
        assert np.array_equal(np.isnan(got), nan)
        bad = np.flatnonzero(got[~nan].view(np.uint32) != ref[~nan].view(np.uint32))
    else:  # the half types' angles take the block-cooperative (pair-major) path
        got = widen(t, orc).reshape(-1)
        assert np.array_equal(np.isnan(got), nan)
        want = narrow_bits(np.ascontiguousarray(ref[~nan]), dtype, orc)
        bad = np.flatnonzero(to_np(t).reshape(-1)[~nan] != want)
    assert bad.size == 0, f"{bad.size} outputs differ; first at {np.flatnonzero(~nan)[bad[:5]].tolist()}"
    if pos_scale == 1.0:
        assert not nan.any()


def test_rope_position_zero_is_identity(dev):
    """rope.rs:196-206: at position 0 the vector is unchanged."""
    x = torch.tensor([1.0, 2.0, 3.0, 4.0], device=dev).view(1, 1, 1, 4)
    ops.rope_(x, None, torch.zeros(1, dtype=torch.int32, device=dev), 1e4)
    assert x.flatten().cpu().tolist() == [1.0, 2.0, 3.0, 4.0]


def test_rope_partial_leaves_tail_unchanged(dev):
    """rope.rs:168-182: head_dim 8, rotary_dim 4, position 3."""
    data = torch.arange(1, 9, dtype=torch.float32, device=dev).view(1, 1, 1, 8)
    x = data.clone()
    ops.rope_(x, None, torch.tensor([3], dtype=torch.int32, device=dev), 1e4, rotary_dim=4)
    assert torch.equal(x[..., 4:], data[..., 4:])
    assert (x[..., :4] - data[..., :4]).abs().max() > 1e-6


def test_rope_interleaved_is_permuted_neox(dev, orc):
    """interleaved(P x) = P neox(x) for the GGUF row permutation P, bit for bit on the GPU."""
    H, S, D = 3, 17, 64
    x = _gen((1, H, S, D), 300, dev)
    pos = torch.arange(S, dtype=torch.int32, device=dev) + 5
    xn = x.clone()
    ops.rope_(xn, None, pos, 1e4)
    # P maps HF channel a*D/2 + b to interleaved channel 2b + a (gguf_weights.rs:111-115)
    perm = torch.tensor([(c % 2) * (D // 2) + c // 2 for c in range(D)], device=dev)
    xi = x[..., perm].contiguous()
    ops.rope_(xi, None, pos, 1e4, interleaved=True)
    assert torch.equal(xi, xn[..., perm])


def test_rope_rejects_bad_arguments(dev):
    from sapient_amd._lib import EINVAL, lib
    L = lib()
    x = torch.zeros(1, 2, 3, 8, device=dev)
    pos = torch.zeros(3, dtype=torch.int32, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    args = lambda D, rd, layout=0: (x.data_ptr(), 2, None, 0, 0, layout, pos.data_ptr(), 1, 3, D, rd, 1e4, 1.0, s)
    assert L.sph_rope(*args(7, 7)) == EINVAL      # odd head_dim
    assert L.sph_rope(*args(8, 10)) == EINVAL     # rotary_dim > head_dim
    assert L.sph_rope(*args(8, 3)) == EINVAL      # odd rotary_dim
    assert L.sph_rope(*args(8, 8, 2)) == EINVAL   # unknown layout
