"""GPU parity: add, mul, SiLU, SwiGLU, GELU (tanh and erf forms) and the
last-dimension bias add against the oracle.

Reference: crates/sapient-backends/cpu/src/kernels/elementwise.rs:27-69 (add/mul and
broadcast), :120-127 (gelu), :135-138 with :163-174 (gelu_erf), :141-143 (silu);
SwiGLU = silu then mul (llama.rs:531-532); bias add
crates/sapient-models/src/forward/common.rs:556-569.

Tolerances:
  add / mul          bit-exact (one IEEE operation, same rounding)
  SiLU / SwiGLU      bit-exact in every dtype: f32 evaluates glibc's own expf
                     algorithm; half types a certified fast path with that
                     expression as the fallback (exhaustive over the gate's
                     16-bit patterns)
  GELU (every dtype) bit-exact: the kernel evaluates glibc's own tanhf algorithm
  erf-GELU (every dtype) bit-exact: glibc's own expf algorithm
  bias add           bit-exact (one IEEE add)
"""
import numpy as np
import pytest
import torch

from helpers import assert_ulp16, assert_bits16_equal, assert_bits_equal, max_rel, narrow_bits, to_np, ulp_diff16, widen
from refvec import WgpuLcg

import sapient_amd.ops as ops

pytestmark = pytest.mark.gpu
DTYPES = [torch.float32, torch.float16, torch.bfloat16]
IDS = lambda d: str(d).split(".")[-1]


def _gen(shape, seed, dev, std=1.0, dtype=torch.float32):
    g = torch.Generator(device=dev).manual_seed(seed)
    return (torch.randn(shape, generator=g, device=dev) * std).to(dtype)


SPECIALS = np.array([0.0, -0.0, 1.0, -1.0, 0.5, -0.5, 3.0, -3.0, 5.0, -5.0, 8.0, -8.0, 10.0, -10.0, 20.0,
                     -20.0, 40.0, -40.0, 79.9, -79.9, -80.0, -80.1, 87.3, -87.3, 88.7, -88.7, -88.73, 89.0,
                     -89.0, 100.0, -100.0, 1e-20, -1e-20, 1e-40, -1e-40, 3.4e38, -3.4e38, np.inf, -np.inf,
                     np.nan], np.float32)


def _check(out, ref32, orc, rtol, what):
    if out.dtype == torch.float32:
        r = max_rel(to_np(out), ref32, floor=1e-37)
        assert r <= rtol, f"{what}: max rel err {r:.3e}"
    else:
        assert_ulp16(to_np(out), narrow_bits(ref32, out.dtype, orc), out.dtype, 1, what)


def test_swiglu_and_add_match_wgpu_test_vectors(dev, orc):
    """resident.rs:103-124: n = 4096, lcg 0x9E3779B9; add ≤ 1e-5, swiglu ≤ 1e-4 abs there."""
    nxt = WgpuLcg()
    a, b = nxt.take(4096), nxt.take(4096)
    ta, tb = torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev)
    print("case add/swiglu wgpu-vectors", flush=True)
    assert_bits_equal(to_np(ops.add(ta, tb)), orc.add(a, b), "add")
    sg = to_np(ops.swiglu(ta, tb))
    assert max_rel(sg, orc.swiglu(a, b), floor=1e-37) <= 1e-5
    silu = a.astype(np.float64) / (1 + np.exp(-a.astype(np.float64)))
    assert np.abs(sg - silu * b).max() < 1e-4


@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
@pytest.mark.parametrize("n", [1, 3, 8, 31, 4096, 4096 * 4864 + 7])
def test_add_mul_bit_exact(dev, orc, dtype, n):
    print(f"case add/mul {dtype} n={n}", flush=True)
    a, b = _gen((n,), 3, dev, dtype=dtype), _gen((n,), 4, dev, dtype=dtype)
    a32, b32 = widen(a, orc), widen(b, orc)
    for fn, ref in ((ops.add, orc.add), (ops.mul, orc.mul)):
        got = fn(a, b)
        want = ref(a32, b32)
        if dtype == torch.float32:
            assert_bits_equal(to_np(got), want, fn.__name__)
        else:
            assert_bits16_equal(to_np(got), narrow_bits(want, dtype, orc), f"{fn.__name__} {dtype}")


def test_add_mul_scalar_broadcast(dev, orc):
    """elementwise.rs:41-48 and the test at :226-231: [1,2,3] * [2] = [2,4,6]."""
    a = torch.tensor([1.0, 2.0, 3.0], device=dev)
    s = torch.tensor([2.0], device=dev)
    assert ops.mul(a, s).cpu().tolist() == [2.0, 4.0, 6.0]
    assert ops.mul(s, a).cpu().tolist() == [2.0, 4.0, 6.0]
    assert ops.add(a, s).cpu().tolist() == [3.0, 4.0, 5.0]
    x = _gen((1000,), 5, dev)
    assert_bits_equal(to_np(ops.add(x, s)), orc.add(to_np(x), np.float32([2.0])), "add broadcast")
    from sapient_amd._lib import EINVAL, SapientHipError
    with pytest.raises(SapientHipError) as e:
        ops.add(a, torch.zeros(2, device=dev))
    assert e.value.status == EINVAL


@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
# 2^22 / 2^22 + 4 (f32) and 2^23 / 2^23 + 8 (half types) straddle the one-vector-per-thread launch of
# small and mid-size element-wise calls (up to 2^20 16-byte vectors; a vector holds 4 f32 or 8 half values);
# 2047 / 2048 and 2^18 / 2^18 + 1 the one-element-per-thread launch of small ones.
@pytest.mark.parametrize("n", [1, 5, 2047, 2048, 4864, 1 << 18, (1 << 18) + 1, 512 * 4864, 1 << 22, (1 << 22) + 4,
                               1 << 23, (1 << 23) + 8])
def test_silu_swiglu(dev, orc, dtype, n):
    print(f"case silu/swiglu {dtype} n={n}", flush=True)
    g, u = _gen((n,), 6, dev, 2.0, dtype), _gen((n,), 7, dev, 2.0, dtype)
    g32, u32 = widen(g, orc), widen(u, orc)
    _exact(ops.silu(g), orc.silu(g32), orc, f"silu {dtype}")
    _exact(ops.swiglu(g, u), orc.swiglu(g32, u32), orc, f"swiglu {dtype}")


def _exact(out: torch.Tensor, ref32: np.ndarray, orc, what: str):
    """Bit-exact against the oracle (half types: its f32 result rounded to nearest-even); NaN
    matches NaN."""
    if out.dtype == torch.float32:
        assert_bits_equal(to_np(out), ref32, what)
    else:
        got, want = to_np(out).reshape(-1), narrow_bits(ref32, out.dtype, orc).reshape(-1)
        nan = np.isnan(ref32.reshape(-1))
        assert_bits16_equal(got[~nan], want[~nan], what)
        assert (ulp_diff16(got[nan], want[nan], out.dtype) == 0).all(), what + " NaN"


# Launches of up to 2^18 elements run one element per thread (half-precision GELU reading its table
# from cache); larger ones take the vector kernels (16-byte accesses, the half types' certified fast
# paths, GELU's table staged per block). The exhaustive tests check the small form against the oracle
# over every 16-bit pattern and then the vector form against it over the same patterns tiled past
# that bound.
TILES = 5  # 5 x 65536 = 327680 > 2^18


def _tiled_same(fn, x: torch.Tensor, got_small: np.ndarray, what: str):
    big = to_np(fn(x.repeat(TILES)))
    assert np.array_equal(big, np.tile(got_small, TILES)), what + " (vector kernels)"


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=IDS)
def test_silu_swiglu_half_exhaustive_bit_exact(dev, orc, dtype):
    """Every 16-bit gate pattern: SiLU, and SwiGLU with up = 1, −3.7, ~N(0, 2), ~N(0, 300) and
    ±tiny — the reference's f32 result rounded once to the half type, bit for bit."""
    g = torch.arange(0, 65536, dtype=torch.int32).to(torch.int16).view(dtype).to(dev)
    g32 = widen(g, orc)
    print(f"case silu/swiglu exhaustive {dtype}", flush=True)
    s = ops.silu(g)
    _exact(s, orc.silu(g32), orc, f"silu {dtype}")
    _tiled_same(ops.silu, g, to_np(s), f"silu {dtype}")
    ups = [torch.ones(65536, device=dev), torch.full((65536,), -3.7, device=dev),
           _gen((65536,), 31, dev, 2.0), _gen((65536,), 32, dev, 300.0), _gen((65536,), 33, dev, 1e-30)]
    for i, u in enumerate(ups):
        u = u.to(dtype)
        y = ops.swiglu(g, u)
        _exact(y, orc.swiglu(g32, widen(u, orc)), orc, f"swiglu {dtype} up #{i}")
        big = to_np(ops.swiglu(g.repeat(TILES), u.repeat(TILES)))
        assert np.array_equal(big, np.tile(to_np(y), TILES)), f"swiglu {dtype} up #{i} (vector kernels)"


def test_silu_special_values(dev, orc):
    x = torch.from_numpy(SPECIALS).to(dev)
    assert_bits_equal(to_np(ops.silu(x)), orc.silu(SPECIALS), "silu specials")


def test_silu_f32_bit_exact_wide_range(dev, orc):
    """f32 SiLU over ~N(0, 30) and a log-uniform magnitude sweep (−104 .. 104, subnormal results
    included): the reference's bits."""
    g = torch.Generator(device=dev).manual_seed(17)
    mags = torch.exp(torch.rand(1 << 20, generator=g, device=dev) * 9.3 - 4.6)
    signs = torch.where(torch.rand(1 << 20, generator=g, device=dev) < 0.5, -1.0, 1.0)
    x = torch.cat([_gen((1 << 20,), 18, dev, 30.0), mags * signs])
    assert_bits_equal(to_np(ops.silu(x)), orc.silu(to_np(x)), "silu f32 wide")


def test_swiglu_f32_full(dev, orc):
    """SwiGLU on [8192, 14336] f32, inputs ~N(0, 2): bit-exact."""
    shape = (8192, 14336)
    print("case swiglu full f32", flush=True)
    g, u = _gen(shape, 53, dev, 2.0), _gen(shape, 54, dev, 2.0)
    out = ops.swiglu(g, u)
    torch.cuda.synchronize()
    assert_bits_equal(to_np(out), orc.swiglu(to_np(g), to_np(u)), "swiglu full f32")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=IDS)
def test_swiglu_llama3_8b_full(dev, orc, dtype):
    """SwiGLU on [8192, 14336] in half types, inputs ~N(0, 2): bit-exact everywhere."""
    shape = (8192, 14336)
    print(f"case swiglu full {dtype}", flush=True)
    g, u = _gen(shape, 51, dev, 2.0, dtype), _gen(shape, 52, dev, 2.0, dtype)
    out = ops.swiglu(g, u)
    torch.cuda.synchronize()
    _exact(out, orc.swiglu(widen(g, orc), widen(u, orc)), orc, f"swiglu full {dtype}")


def test_swiglu_in_place(dev, orc):
    g, u = _gen((4099,), 8, dev, 2.0), _gen((4099,), 9, dev, 2.0)
    want = orc.swiglu(to_np(g), to_np(u))
    ops.swiglu(g, u, out=g)
    assert max_rel(to_np(g), want, floor=1e-37) <= 1e-5


def test_gelu_f32_bit_exact(dev, orc):
    """f32 GELU reproduces glibc's tanhf bits, so the result equals the oracle exactly."""
    x = torch.cat([_gen((1 << 20,), 10, dev, 2.0), _gen((1 << 16,), 11, dev, 8.0), torch.from_numpy(SPECIALS).to(dev)])
    print("case gelu f32", flush=True)
    want = orc.gelu(to_np(x))
    assert_bits_equal(to_np(ops.gelu_tanh(x)), want, "gelu f32")
    # the one-element-per-thread launch of small calls (up to 2^18 elements), on slices of the same inputs
    for lo, hi in ((0, 4864), (5, 1 << 18), ((1 << 20) - 7, (1 << 20) + 70000)):
        assert_bits_equal(to_np(ops.gelu_tanh(x[lo:hi])), want[lo:hi], f"gelu f32 [{lo}:{hi}]")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=IDS)
def test_gelu_half_exhaustive_bit_exact(dev, orc, dtype):
    """Every one of the 65536 f16 / bf16 inputs: output bits equal RNE(oracle(widen(x)))."""
    bits = torch.arange(0, 65536, dtype=torch.int32).to(torch.int16).view(dtype)
    x = bits.to(dev)
    print(f"case gelu exhaustive {dtype}", flush=True)
    got = to_np(ops.gelu_tanh(x))
    want = narrow_bits(orc.gelu(widen(x, orc)), dtype, orc)
    nan = np.isnan(orc.gelu(widen(x, orc)))
    assert_bits16_equal(got[~nan], want[~nan], f"gelu {dtype}")
    assert (ulp_diff16(got[nan], want[nan], dtype) == 0).all()
    # unaligned / tail path gives the same bits
    got2 = to_np(ops.gelu_tanh(x[3:]))
    assert np.array_equal(got2, got[3:])
    _tiled_same(ops.gelu_tanh, x, got, f"gelu {dtype}")


def test_gelu_phi2_full(dev, orc):
    """GELU-tanh on [8192, 10240] f16 (phi-2 FFN), inputs ~N(0, 2): bit-exact."""
    x = _gen((8192, 10240), 61, dev, 2.0, torch.float16)
    print("case gelu full f16", flush=True)
    out = ops.gelu_tanh(x)
    torch.cuda.synchronize()
    want = narrow_bits(orc.gelu(widen(x, orc)), torch.float16, orc)
    assert_bits16_equal(to_np(out), want, "gelu full f16")


def test_gelu_kat(dev):
    """elementwise.rs:206-210: gelu(0) = 0."""
    assert ops.gelu_tanh(torch.zeros(1, device=dev)).item() == 0.0


def test_gelu_erf_f32_bit_exact(dev, orc):
    """f32 erf-GELU reproduces glibc's expf bits, so the result equals the oracle exactly."""
    x = torch.cat([_gen((1 << 20,), 12, dev, 2.0), _gen((1 << 16,), 13, dev, 8.0), torch.from_numpy(SPECIALS).to(dev)])
    print("case gelu_erf f32", flush=True)
    assert_bits_equal(to_np(ops.gelu_erf(x)), orc.gelu_erf(to_np(x)), "gelu_erf f32")


def test_gelu_erf_matches_wgpu_test_vectors(dev, orc):
    """wgpu tests/resident.rs:909-930: n = 4096 + 37, lcg · 4; the reference test's bound is 1e-5."""
    x = WgpuLcg().take(4096 + 37) * np.float32(4.0)
    got = to_np(ops.gelu_erf(torch.from_numpy(x).to(dev)))
    assert_bits_equal(got, orc.gelu_erf(x), "gelu_erf wgpu vectors")
    from math import erf
    want = np.array([0.5 * t * (1 + erf(t / np.sqrt(2))) for t in x.astype(np.float64)])
    assert np.abs(got - want).max() < 1e-5


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=IDS)
def test_gelu_erf_half_exhaustive_bit_exact(dev, orc, dtype):
    """Every one of the 65536 f16 / bf16 inputs: output bits equal RNE(oracle(widen(x)))."""
    bits = torch.arange(0, 65536, dtype=torch.int32).to(torch.int16).view(dtype)
    x = bits.to(dev)
    print(f"case gelu_erf exhaustive {dtype}", flush=True)
    got = to_np(ops.gelu_erf(x))
    ref = orc.gelu_erf(widen(x, orc))
    want = narrow_bits(ref, dtype, orc)
    nan = np.isnan(ref)
    assert_bits16_equal(got[~nan], want[~nan], f"gelu_erf {dtype}")
    assert (ulp_diff16(got[nan], want[nan], dtype) == 0).all()
    got2 = to_np(ops.gelu_erf(x[3:]))
    assert np.array_equal(got2, got[3:])
    _tiled_same(ops.gelu_erf, x, got, f"gelu_erf {dtype}")


@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
def test_gelu_erf_whisper_full(dev, orc, dtype):
    """erf-GELU on [1500 · 8, 5120] (Whisper-large FFN width, 8 utterances), inputs ~N(0, 2): bit-exact."""
    x = _gen((12000, 5120), 62, dev, 2.0, dtype)
    print(f"case gelu_erf full {dtype}", flush=True)
    out = ops.gelu_erf(x)
    torch.cuda.synchronize()
    ref = orc.gelu_erf(widen(x, orc))
    if dtype == torch.float32:
        assert_bits_equal(to_np(out), ref, "gelu_erf full f32")
    else:
        assert_bits16_equal(to_np(out), narrow_bits(ref, dtype, orc), f"gelu_erf full {dtype}")


def test_gelu_erf_kat(dev):
    """elementwise.rs:216-224: g(0) = 0, g(1) = 0.8413447, g(-1) = -0.1586553 within 1e-4."""
    v = ops.gelu_erf(torch.tensor([0.0, 1.0, -1.0], device=dev)).cpu().numpy()
    assert abs(v[0]) < 1e-6 and abs(v[1] - 0.8413447) < 1e-4 and abs(v[2] + 0.1586553) < 1e-4


@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
@pytest.mark.parametrize("bdtype", DTYPES, ids=IDS)
@pytest.mark.parametrize("rows,n", [(13, 320), (1, 1), (5, 3), (7, 100), (64, 1280), (3, 4096), (2, 8200),
                                    (1, 65536)])
def test_add_bias_bit_exact(dev, orc, dtype, bdtype, rows, n):
    print(f"case add_bias {dtype} bias {bdtype} {rows}x{n}", flush=True)
    y = _gen((rows, n), 20 + n, dev, dtype=dtype)
    bias = _gen((n,), 21, dev, dtype=bdtype)
    got = ops.add_bias(y, bias)
    want = orc.add_bias_last_dim(widen(y, orc), widen(bias, orc))
    if dtype == torch.float32:
        assert_bits_equal(to_np(got), want, "add_bias")
    else:
        assert_bits16_equal(to_np(got), narrow_bits(want, dtype, orc), f"add_bias {dtype}")


def test_add_bias_matches_wgpu_test_vectors(dev, orc):
    """wgpu tests/resident.rs:933-951: 13 x 320, lcg; the reference test's bound is 1e-5."""
    nxt = WgpuLcg()
    x = nxt.take(13 * 320).reshape(13, 320)
    bias = nxt.take(320)
    got = to_np(ops.add_bias(torch.from_numpy(x).to(dev), torch.from_numpy(bias).to(dev)))
    assert_bits_equal(got, orc.add_bias_last_dim(x, bias), "add_bias wgpu vectors")
    assert np.abs(got - (x + bias)).max() < 1e-5


def test_add_bias_full_in_place_and_unaligned(dev, orc):
    """16384 x 4096 f32 with an f16 bias (the reference's F32-y / half-bias case), in place; then
    4-byte-offset views through the scalar path."""
    y = _gen((16384, 4096), 31, dev)
    bias = _gen((4096,), 32, dev, dtype=torch.float16)
    want = orc.add_bias_last_dim(to_np(y), widen(bias, orc))
    ops.add_bias(y, bias, out=y)
    torch.cuda.synchronize()
    assert_bits_equal(to_np(y), want, "add_bias full in place")
    base = _gen((3 * 640 + 1,), 33, dev)
    yv = base[1:].view(3, 640)
    bb = _gen((641,), 34, dev)[1:]
    got = ops.add_bias(yv, bb)
    assert_bits_equal(to_np(got), orc.add_bias_last_dim(to_np(yv), to_np(bb)), "add_bias unaligned")


def test_add_bias_rejects_bad_arguments(dev):
    from sapient_amd._lib import EINVAL, lib
    L = lib()
    y = torch.zeros(4, 8, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    p = y.data_ptr()
    assert L.sph_add_bias(p, p, 0, p, 0, 32, 5, s) == EINVAL    # total not a multiple of n
    assert L.sph_add_bias(p, p, 0, p, 0, 32, 0, s) == EINVAL    # n = 0 with data
    assert L.sph_add_bias(p, p, 8, p, 0, 32, 8, s) == EINVAL    # bias dtype
    assert L.sph_add_bias(p, None, 0, p, 0, 32, 8, s) == EINVAL  # null bias
    assert L.sph_add_bias(p, p, 0, p, 0, 0, 8, s) == 0           # empty is a no-op
    with pytest.raises(ValueError, match="does not match last dim"):
        ops.add_bias(y, torch.zeros(7, device=dev))
