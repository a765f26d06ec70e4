"""Pins the CPU oracle before the GPU results are held to it (no GPU needed).

Each oracle function is held to something it was not written from:
  - the known-answer tests in the reference's own test modules,
  - the reference tests' in-test restatements and generators (tests/refvec.py),
  - closed forms in float64 and exact invariants,
  - exhaustive sweeps (half-precision conversions over all inputs),
chosen so that a dropped term, a wrong sign or index, or a transposed operand
fails at least one of them.
"""
import concurrent.futures as cf
import ctypes
import ctypes.util

import numpy as np
import pytest
import torch

import oracle
from refvec import (WgpuLcg, f16_bits, gather_test_values, quantize_q8_0_blocks, random_q4_k_blocks,
                    random_q6_k_blocks)


def _bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


# ───────────────────────── half-precision conversions ─────────────────────────
def test_f16_widening_all_patterns():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.f16_bits_to_f32(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(_bits(got)[~nan], _bits(want)[~nan])
    assert np.isnan(got[nan]).all()
    assert ((_bits(got[nan]) & 0x400000) != 0).all()  # half's widening returns quiet NaNs


def test_bf16_widening_all_patterns():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.bf16_bits_to_f32(h)
    want = torch.from_numpy(h.view(np.int16).copy()).view(torch.bfloat16).float().numpy()
    nan = np.isnan(want)
    assert np.array_equal(_bits(got)[~nan], _bits(want)[~nan])
    assert np.isnan(got[nan]).all()


def _sweep(check, chunk_bits=20):
    """Run check(lo, hi) over all 2^32 f32 patterns in parallel chunks."""
    n = 1 << 32
    step = 1 << chunk_bits
    with cf.ThreadPoolExecutor(8) as ex:
        bad = sum(ex.map(lambda lo: check(lo, lo + step), range(0, n, step)))
    return bad


def test_f16_narrowing_exhaustive_matches_ieee_rne():
    """All 2^32 f32 inputs: oracle f32→f16 equals the x86 F16C conversion (torch's f32 → f16 on the
    CPU, IEEE round-to-nearest-even; NaN: NaN with the quiet bit, as half's from_f32)."""
    def check(lo, hi):
        x = np.arange(lo, hi, dtype=np.uint32).view(np.float32)
        got = oracle.f32_to_f16_bits(x)
        want = torch.from_numpy(x).to(torch.float16).view(torch.int16).numpy().view(np.uint16)
        nan = np.isnan(x)
        ok = (got == want) | (nan & ((got & 0x7E00) == 0x7E00))
        return int((~ok).sum())
    assert _sweep(check) == 0


def test_f16_narrowing_references_agree_on_a_sample():
    """The exhaustive test's reference (torch / F16C) against numpy's software IEEE conversion, a
    second implementation, on every 97th f32 pattern (44 M inputs, every exponent and class):
    equal on every non-NaN input; on NaNs F16C sets the quiet bit and numpy returns a NaN."""
    x = (np.arange(0, (1 << 32) // 97, dtype=np.uint32) * np.uint32(97)).view(np.float32)
    a = torch.from_numpy(x).to(torch.float16).view(torch.int16).numpy().view(np.uint16)
    with np.errstate(over="ignore"):
        b = x.astype(np.float16).view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(a[~nan], b[~nan])
    assert ((a[nan] & 0x7E00) == 0x7E00).all()
    assert ((b[nan] & 0x7C00) == 0x7C00).all() and ((b[nan] & 0x03FF) != 0).all()


def test_bf16_narrowing_exhaustive_matches_ieee_rne():
    """All 2^32 f32 inputs: oracle f32→bf16 equals torch's round-to-nearest-even conversion."""
    def check(lo, hi):
        x = np.arange(lo, hi, dtype=np.uint32).view(np.float32)
        got = oracle.f32_to_bf16_bits(x)
        want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
        nan = np.isnan(x)
        ok = (got == want) | (nan & ((got & 0x7FC0) == 0x7FC0))
        return int((~ok).sum())
    assert _sweep(check) == 0


# ───────────────────────────────── RMSNorm ─────────────────────────────────
def test_rms_norm_kat():
    """layernorm.rs:126-149: [3, 4], w = 1, eps = 0 → [3, 4] / sqrt(12.5) within 1e-5."""
    y = oracle.rms_norm(np.array([[3.0, 4.0]], np.float32), np.ones(2, np.float32), 0.0)
    e = np.float32(12.5) ** np.float32(0.5)
    assert abs(y[0, 0] - np.float32(3.0) / e) < 1e-5 and abs(y[0, 1] - np.float32(4.0) / e) < 1e-5


def test_rms_norm_serial_fold_bit_exact():
    """Bit-exact against a numpy restatement of the reference's op order:
    sequential f32 fold of v*v (Iterator::sum), / dim, 1/sqrt(+eps), (x*inv)*w."""
    rng = np.random.default_rng(1)
    x = rng.standard_normal((64, 896), dtype=np.float32)
    w = (rng.standard_normal(896, dtype=np.float32) * np.float32(0.1) + np.float32(1.0)).astype(np.float32)
    sq = (x * x).astype(np.float32)
    acc = np.add.accumulate(sq, axis=1, dtype=np.float32)[:, -1]
    inv = (np.float32(1.0) / np.sqrt(acc / np.float32(896) + np.float32(1e-6))).astype(np.float32)
    want = ((x * inv[:, None]).astype(np.float32) * w).astype(np.float32)
    assert np.array_equal(_bits(oracle.rms_norm(x, w, 1e-6)), _bits(want))


def test_rms_norm_closed_form_and_invariants():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((32, 4096), dtype=np.float32)
    w = rng.standard_normal(4096, dtype=np.float32)
    y = oracle.rms_norm(x, w, 1e-5)
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + 1e-5) * w
    assert np.max(np.abs(y - want) / np.abs(want)) < 1e-5
    # power-of-two scaling is exact at eps = 0: y(4x) == y(x) bit for bit
    assert np.array_equal(_bits(oracle.rms_norm(4 * x, w, 0.0)), _bits(oracle.rms_norm(x, w, 0.0)))
    # unit weight: every row has mean square 1
    u = oracle.rms_norm(x, np.ones(4096, np.float32), 0.0).astype(np.float64)
    assert np.allclose((u ** 2).mean(axis=1), 1.0, atol=1e-5)
    # None weight equals unit weight
    assert np.array_equal(oracle.rms_norm(x, None, 1e-5), oracle.rms_norm(x, np.ones(4096, np.float32), 1e-5))


def test_rms_norm_matches_wgpu_test_restatement():
    """resident.rs:15-59: 5 x 1536, seed 0x12345678, w = 0.5 + |next()|, eps 1e-5, ≤ 1e-4 abs."""
    nxt = WgpuLcg(0x12345678)
    x = nxt.take(5 * 1536).reshape(5, 1536)
    w = np.float32(0.5) + np.abs(nxt.take(1536))
    ms = (x * x).sum(axis=1, dtype=np.float32) / np.float32(1536)
    want = x * (np.float32(1.0) / np.sqrt(ms + np.float32(1e-5)))[:, None] * w
    assert np.abs(oracle.rms_norm(x, w, 1e-5) - want).max() < 1e-4


def test_layer_norm_kat():
    """layernorm.rs:113-123: [[1, 2], [3, 4]], no weight / bias, eps 1e-5 → ±1 within 1e-4."""
    y = oracle.layer_norm(np.array([[1.0, 2.0], [3.0, 4.0]], np.float32), None, None, 1e-5)
    assert np.abs(y - np.array([[-1, 1], [-1, 1]], np.float32)).max() < 1e-4


def test_layer_norm_serial_two_pass_bit_exact():
    """Bit-exact against a numpy restatement of the reference's op order: f32
    serial folds of x and of (x - mean)^2, each / n, 1/sqrt(var + eps), then
    (x - mean) * inv * w + b."""
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((16, 768)) * 3 + 0.5).astype(np.float32)
    w = (np.float32(0.5) + np.abs(rng.standard_normal(768))).astype(np.float32)
    b = (rng.standard_normal(768) * 0.1).astype(np.float32)
    n = np.float32(768)
    mean = np.add.accumulate(x, axis=1, dtype=np.float32)[:, -1] / n
    d = (x - mean[:, None]).astype(np.float32)
    var = np.add.accumulate((d * d).astype(np.float32), axis=1, dtype=np.float32)[:, -1] / n
    inv = (np.float32(1.0) / np.sqrt((var + np.float32(1e-5)).astype(np.float32))).astype(np.float32)
    normed = (d * inv[:, None]).astype(np.float32)
    assert np.array_equal(_bits(oracle.layer_norm(x, w, b, 1e-5)), _bits(((normed * w).astype(np.float32) + b)))
    assert np.array_equal(_bits(oracle.layer_norm(x, w, None, 1e-5)), _bits((normed * w).astype(np.float32)))
    assert np.array_equal(_bits(oracle.layer_norm(x, None, b, 1e-5)), _bits((normed + b).astype(np.float32)))
    assert np.array_equal(_bits(oracle.layer_norm(x, None, None, 1e-5)), _bits(normed))


def test_layer_norm_closed_form_and_invariants():
    """Against float64 math (population variance, eps inside the root); shift
    invariance; unit weight gives rows of mean 0 and variance 1 / (1 + eps/var)."""
    rng = np.random.default_rng(12)
    x = (rng.standard_normal((32, 4096)) * 2 + 3).astype(np.float32)
    w = rng.standard_normal(4096).astype(np.float32)
    b = rng.standard_normal(4096).astype(np.float32)
    x64 = x.astype(np.float64)
    mu = x64.mean(axis=1, keepdims=True)
    var = x64.var(axis=1, keepdims=True)  # population variance, divides by n
    want = (x64 - mu) / np.sqrt(var + 1e-5) * w + b
    y = oracle.layer_norm(x, w, b, 1e-5).astype(np.float64)
    # The serial f32 sums move mean and variance by ~1e-6 relative: an error of
    # |w| · 2e-5 · (1 + |normed|) at most. A variance divided by n - 1 would
    # shift normed by 1.2e-4 · |normed| and fail.
    normed = np.abs((x64 - mu) / np.sqrt(var))
    assert (np.abs(y - want) <= np.abs(w) * 2e-5 * (1 + normed) + np.abs(b) * 2.0 ** -22).all()
    n1 = (x64 - mu) / np.sqrt(x64.var(axis=1, ddof=1, keepdims=True) + 1e-5) * w + b
    assert not (np.abs(n1 - want) <= np.abs(w) * 2e-5 * (1 + normed) + np.abs(b) * 2.0 ** -22).all()
    # a large eps is visible (pins where eps enters)
    big = (x64 - mu) / np.sqrt(var + 4.0)
    assert np.abs(oracle.layer_norm(x, None, None, 4.0) - big).max() < 1e-5
    # unit weight, zero bias: mean 0, variance var / (var + eps)
    u = oracle.layer_norm(x, None, None, 1e-5).astype(np.float64)
    assert np.abs(u.mean(axis=1)).max() < 1e-5
    assert np.allclose(u.var(axis=1), (var / (var + 1e-5))[:, 0], atol=1e-5)


def test_layer_norm_matches_wgpu_test_restatement():
    """wgpu tests/resident.rs:860-886: 7 x 1536, lcg * 3, w = 0.5 + |next()|, b = next() * 0.1, eps 1e-5,
    max |Δ| < 1e-4 against the test's own f32 restatement (:838-857)."""
    nxt = WgpuLcg()
    x = (nxt.take(7 * 1536) * np.float32(3.0)).reshape(7, 1536)
    w = np.float32(0.5) + np.abs(nxt.take(1536))
    b = nxt.take(1536) * np.float32(0.1)
    mean = x.sum(axis=1, dtype=np.float32) / np.float32(1536)
    var = ((x - mean[:, None]) ** 2).sum(axis=1, dtype=np.float32) / np.float32(1536)
    want = (x - mean[:, None]) * (np.float32(1.0) / np.sqrt(var + np.float32(1e-5)))[:, None] * w + b
    assert np.abs(oracle.layer_norm(x, w, b, 1e-5) - want).max() < 1e-4


def test_add_bias_last_dim():
    """common.rs:556-569: bias[i % n] added to every row, exactly (integer-valued
    data makes every sum exact); a length mismatch is an error; wgpu
    tests/resident.rs:933-951 data (13 x 320) within 1e-5."""
    y = np.arange(12, dtype=np.float32).reshape(2, 2, 3)
    out = oracle.add_bias_last_dim(y, np.float32([100, 200, 300]))
    assert np.array_equal(out, y + np.float32([100, 200, 300]))
    with pytest.raises(ValueError, match="does not match last dim"):
        oracle.add_bias_last_dim(y, np.float32([1, 2]))
    nxt = WgpuLcg()
    x = nxt.take(13 * 320).reshape(13, 320)
    bias = nxt.take(320)
    assert np.abs(oracle.add_bias_last_dim(x, bias) - (x + bias)).max() < 1e-5
    assert np.array_equal(_bits(oracle.add_bias_last_dim(x, bias)), _bits((x + bias).astype(np.float32)))


def test_add_rms_norm_is_add_then_rms_norm():
    rng = np.random.default_rng(3)
    x, r = rng.standard_normal((2, 8, 256), dtype=np.float32)
    w = rng.standard_normal(256, dtype=np.float32)
    y, r2 = oracle.add_rms_norm(x, r, w, 1e-5)
    assert np.array_equal(_bits(r2), _bits((x + r).astype(np.float32)))
    assert np.array_equal(_bits(y), _bits(oracle.rms_norm(x + r, w, 1e-5)))
    # no weight is unit weight, as for rms_norm; a weight of the wrong length is refused
    y1, _ = oracle.add_rms_norm(x, r, None, 1e-5)
    assert np.array_equal(_bits(y1), _bits(oracle.add_rms_norm(x, r, np.ones(256, np.float32), 1e-5)[0]))
    with pytest.raises(ValueError):
        oracle.add_rms_norm(x, r, w[:255], 1e-5)


# ─────────────────────────────── add / mul ───────────────────────────────
def test_add_mul_and_broadcast():
    """elementwise.rs:184-194 (add KAT) and :226-231 (scalar broadcast)."""
    assert abs(oracle.add(np.float32([1, 2]), np.float32([3, 4]))[0] - 4.0) < 1e-6
    assert oracle.mul(np.float32([1, 2, 3]), np.float32([2])).tolist() == [2.0, 4.0, 6.0]
    assert oracle.mul(np.float32([2]), np.float32([1, 2, 3])).tolist() == [2.0, 4.0, 6.0]
    rng = np.random.default_rng(4)
    a, b = rng.standard_normal((2, 1000), dtype=np.float32)
    assert np.array_equal(_bits(oracle.add(a, b)), _bits(a + b))
    assert np.array_equal(_bits(oracle.mul(a, b)), _bits(a * b))
    with pytest.raises(oracle.OracleError):
        oracle.add(np.zeros(3, np.float32), np.zeros(2, np.float32))


# ─────────────────────────────── SiLU / SwiGLU ───────────────────────────────
def test_silu_swiglu_closed_form():
    rng = np.random.default_rng(5)
    g = (rng.standard_normal(1 << 16) * 4).astype(np.float32)
    u = rng.standard_normal(1 << 16).astype(np.float32)
    g64 = g.astype(np.float64)
    s64 = g64 / (1 + np.exp(-g64))
    s = oracle.silu(g)
    assert np.max(np.abs(s - s64) / np.maximum(np.abs(s64), 1e-300)) < 4e-7  # ≤ ~3 f32 roundings
    assert np.array_equal(_bits(oracle.swiglu(g, u)), _bits((s * u).astype(np.float32)))


def test_silu_special_values():
    x = np.float32([0.0, -0.0, np.inf, -np.inf, np.nan, -100.0, 100.0, -88.8])
    s = oracle.silu(x)
    assert s[0] == 0 and np.signbit(s[1]) and s[2] == np.inf
    assert np.isnan(s[3]) and np.isnan(s[4])          # -inf / inf and NaN
    assert s[5] == 0 and np.signbit(s[5])             # expf(100) overflows: -100 / inf = -0
    assert s[6] == np.float32(100.0) and s[7] == 0


def test_swiglu_matches_wgpu_test_restatement():
    """resident.rs:103-124: n = 4096, lcg 0x9E3779B9, |swiglu - silu(a)·b| < 1e-4."""
    nxt = WgpuLcg()
    a, b = nxt.take(4096), nxt.take(4096)
    silu = a * (np.float32(1.0) / (np.float32(1.0) + np.exp(-a)))
    assert np.abs(oracle.swiglu(a, b) - silu * b).max() < 1e-4


# ────────────────────────────────── GELU ──────────────────────────────────
def test_gelu_kats():
    """elementwise.rs:206-210 gelu(0) = 0; :216-224 gelu_erf(0, 1, -1)."""
    assert oracle.gelu(np.float32([0.0]))[0] == 0.0
    g = oracle.gelu_erf(np.float32([0.0, 1.0, -1.0]))
    assert abs(g[0]) < 1e-6 and abs(g[1] - 0.8413447) < 1e-4 and abs(g[2] + 0.1586553) < 1e-4


def test_gelu_closed_form_including_cancellation():
    """Against float64 math: relative 1e-6 where 1 + tanh does not cancel
    (inner > -0.5); elsewhere the f32 result may only differ by the rounding of
    tanh near -1, i.e. |Δ| ≤ |0.5 v| · 2 ulp(1) + 2 ulp of the result."""
    rng = np.random.default_rng(6)
    v = (rng.standard_normal(1 << 18) * 2).astype(np.float32)
    y = oracle.gelu(v).astype(np.float64)
    v64 = v.astype(np.float64)
    inner = 0.7978845608028654 * (v64 + 0.044715 * v64 ** 3)
    y64 = 0.5 * v64 * (1 + np.tanh(inner))
    calm = inner > -0.5
    assert np.max(np.abs(y - y64)[calm] / np.maximum(np.abs(y64[calm]), 1e-30)) < 1e-6
    bound = np.abs(0.5 * v64) * 2.0 ** -22 + np.abs(y64) * 2.0 ** -22 + 1e-45
    assert (np.abs(y - y64)[~calm] <= bound[~calm]).all()


def test_gelu_erf_abramowitz_stegun_bound():
    """erf_approx is A&S 7.1.26 (max error 1.5e-7): against float64 erf over a
    dense grid the oracle stays within 0.5|v| (1.5e-7 + 8 ulp(1)) + 2 ulp(y); a
    wrong coefficient or a dropped term breaks the bound by orders of magnitude.
    Odd symmetry of erf: gelu_erf(v) - gelu_erf(-v) = v up to rounding."""
    from math import erf
    v = np.linspace(-6, 6, 200001, dtype=np.float32)
    y = oracle.gelu_erf(v).astype(np.float64)
    v64 = v.astype(np.float64)
    want = 0.5 * v64 * (1 + np.array([erf(t / np.sqrt(2)) for t in v64]))
    bound = 0.5 * np.abs(v64) * (1.5e-7 + 8 * 2.0 ** -23) + np.abs(want) * 2.0 ** -22 + 1e-45
    assert (np.abs(y - want) <= bound).all()
    ym = oracle.gelu_erf(-v).astype(np.float64)
    assert np.max(np.abs((y - ym) - v64)) < 1e-5 * 6


def test_gelu_erf_matches_wgpu_test_bound():
    """resident.rs:909-930 data: lcg * 4, n = 4133 (erf-GELU next-row op)."""
    x = WgpuLcg().take(4096 + 37) * np.float32(4.0)
    x64 = x.astype(np.float64)
    from math import erf
    want = np.array([0.5 * t * (1 + erf(t / np.sqrt(2))) for t in x64])
    assert np.abs(oracle.gelu_erf(x) - want).max() < 1e-5


# ─────────────────────────────────── RoPE ───────────────────────────────────
_LIBM = ctypes.CDLL(ctypes.util.find_library("m"))
_LIBM.powf.restype = ctypes.c_float
_LIBM.powf.argtypes = [ctypes.c_float, ctypes.c_float]


def _rope64(x, positions, base, rd, pos_scale=1.0, interleaved=False):
    """RoPE with the reference's f32 angle rotated in f64. The denominators come
    from libm's powf — the function Rust's f32::powf binds to — because one ulp
    of powf moves the angle at position 8191 by ~5e-4 rad."""
    half = rd // 2
    i = np.arange(half, dtype=np.float32)
    e = (np.float32(2.0) * i / np.float32(rd)).astype(np.float32)
    den = np.array([_LIBM.powf(float(np.float32(base)), float(v)) for v in e], np.float32)
    p = (np.asarray(positions, np.float32) / np.float32(pos_scale)).astype(np.float32)
    freq = (p[:, None] / den[None, :]).astype(np.float32).astype(np.float64)
    c, s = np.cos(freq), np.sin(freq)
    out = x.astype(np.float64).copy()
    if interleaved:
        x0, x1 = out[..., 0:rd:2].copy(), out[..., 1:rd:2].copy()
        out[..., 0:rd:2], out[..., 1:rd:2] = x0 * c - x1 * s, x1 * c + x0 * s
    else:
        x0, x1 = out[..., :half].copy(), out[..., half:rd].copy()
        out[..., :half], out[..., half:rd] = x0 * c - x1 * s, x1 * c + x0 * s
    return out


@pytest.mark.parametrize("interleaved", [False, True])
def test_rope_closed_form(interleaved):
    rng = np.random.default_rng(7)
    x = rng.standard_normal((2, 3, 50, 64), dtype=np.float32)
    pos = rng.integers(0, 8192, 50)
    got = oracle.apply_rope_partial_scaled(x, pos, 5e5, 64, 1.0, interleaved)
    want = _rope64(x, pos, 5e5, 64, interleaved=interleaved)
    assert np.abs(got - want).max() < 1e-6 * np.abs(x).max() * 4


def test_rope_reference_kats():
    """rope.rs:159-206: output shape, position 0 identity, partial == full, tail unchanged."""
    x = np.full((1, 2, 4, 8), 0.1, np.float32)
    assert oracle.apply_rope(x, list(range(4)), 1e4).shape == (1, 2, 4, 8)
    d = np.float32([1, 2, 3, 4]).reshape(1, 1, 1, 4)
    assert np.abs(oracle.apply_rope(d, [0], 1e4) - d).max() < 1e-6
    data = (np.arange(16, dtype=np.float32) * np.float32(0.1)).reshape(1, 1, 2, 8)
    assert np.abs(oracle.apply_rope(data, [2, 5], 1e4) - oracle.apply_rope_partial_scaled(data, [2, 5], 1e4, 8)).max() < 1e-6
    t = np.arange(1, 9, dtype=np.float32).reshape(1, 1, 1, 8)
    o = oracle.apply_rope_partial_scaled(t, [3], 1e4, 4)
    assert np.array_equal(o[..., 4:], t[..., 4:]) and np.abs(o[..., :4] - t[..., :4]).max() > 1e-6
    with pytest.raises(oracle.OracleError):
        oracle.apply_rope(np.zeros((1, 1, 1, 5), np.float32), [0], 1e4)      # odd head_dim
    with pytest.raises(oracle.OracleError):
        oracle.apply_rope(np.zeros((1, 1, 2, 4), np.float32), [0], 1e4)      # positions != seq


def test_rope_partial_full_matches_apply_rope_bit_exact():
    x = np.random.default_rng(8).standard_normal((1, 4, 9, 128), dtype=np.float32)
    pos = list(range(100, 109))
    assert np.array_equal(_bits(oracle.apply_rope(x, pos, 5e5)),
                          _bits(oracle.apply_rope_partial_scaled(x, pos, 5e5, 128, 1.0)))


def test_unpermute_qk_kat():
    """gguf_weights.rs:458-496: llama.cpp's permutation then unpermute recovers HF rows."""
    n_head, head_dim, hidden = 3, 4, 5
    hf = np.array([[r * 100 + c for c in range(hidden)] for r in range(n_head * head_dim)], np.float32)
    gguf = np.empty_like(hf)
    for h in range(n_head):
        for a in range(2):
            for b in range(head_dim // 2):
                gguf[h * head_dim + b * 2 + a] = hf[h * head_dim + a * head_dim // 2 + b]
    assert np.array_equal(oracle.unpermute_qk_rows(gguf, n_head, head_dim), hf)


def test_rope_interleaved_is_permuted_neox_bit_exact():
    """interleaved(P x) = P neox(x) with P the GGUF q/k row permutation, for every head."""
    B, H, S, D = 1, 4, 11, 64
    x = np.random.default_rng(9).standard_normal((B, H, S, D), dtype=np.float32)
    pos = list(range(1000, 1011))
    neox = oracle.apply_rope_partial_scaled(x, pos, 1e4, D)
    perm = np.array([(c % 2) * (D // 2) + c // 2 for c in range(D)])
    # the same P expressed through the reference's row map on a [H*D, S] view
    xi = oracle.unpermute_qk_rows(x.transpose(0, 1, 3, 2).reshape(H * D, S).copy(), H, D)
    assert np.array_equal(xi.reshape(H, D, S).transpose(0, 2, 1)[None][..., perm], x)
    il = oracle.apply_rope_partial_scaled(x[..., perm], pos, 1e4, D, 1.0, interleaved=True)
    assert np.array_equal(_bits(il), _bits(neox[..., perm]))


# ───────────────────────────── dequant / gather ─────────────────────────────
def test_q8_0_matches_reference_test_quantizer():
    """resident.rs:506-524 / quant.rs:223-235: bytes and dequantized values bit-exact."""
    table = WgpuLcg().take(100 * 320)
    blocks, deq = quantize_q8_0_blocks(table)
    assert np.array_equal(oracle.quantize_q8_0(table), blocks)
    assert np.array_equal(_bits(oracle.dequant(blocks, oracle.Q8_0, table.size)), _bits(deq))


def test_q8_0_every_quant_value_exact():
    scales = np.array([0x0001, 0x03FF, 0x3C00, 0xBC00, 0x7BFF, 0x2E66], np.uint16)
    for sc in scales:
        blocks = np.zeros((8, 34), np.uint8)
        blocks[:, 0:2] = np.array([sc], np.uint16).view(np.uint8)
        blocks[:, 2:] = np.arange(256, dtype=np.uint32).astype(np.uint8).reshape(8, 32)
        got = oracle.dequant(blocks, oracle.Q8_0, 256)
        want = (np.arange(256).astype(np.uint8).view(np.int8).astype(np.float64)
                * float(np.array([sc], np.uint16).view(np.float16)[0]))
        assert np.array_equal(got.astype(np.float64), want)


def test_q4_k_matches_reference_test_generator():
    """resident.rs:600-640: random_q4_k_blocks' own dequant formula, bit-exact."""
    blocks, deq = random_q4_k_blocks(200, WgpuLcg())
    assert np.array_equal(_bits(oracle.dequant(blocks, oracle.Q4_K, 200 * 256)), _bits(deq))


def _q4k_gguf_layout(blocks: np.ndarray) -> np.ndarray:
    """crates/sapient-io/src/gguf.rs:357-389 (dequantize_q4_k), restated with numpy:
    per 64-element group j: 32 low nibbles with (d·sc(2j), dmin·m(2j)), then 32 high
    nibbles with (d·sc(2j+1), dmin·m(2j+1))."""
    b = blocks.reshape(-1, 144)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float32)[:, 0]
    dm = b[:, 2:4].copy().view(np.float16).astype(np.float32)[:, 0]
    s = b[:, 4:16].astype(np.uint32)
    sc = np.empty((b.shape[0], 8), np.uint32)
    mn = np.empty((b.shape[0], 8), np.uint32)
    sc[:, :4], mn[:, :4] = s[:, 0:4] & 63, s[:, 4:8] & 63
    sc[:, 4:] = (s[:, 8:12] & 0xF) | ((s[:, 0:4] >> 6) << 4)
    mn[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    qs = b[:, 16:144].reshape(-1, 4, 32)
    out = np.empty((b.shape[0], 4, 2, 32), np.float32)
    for j in range(4):
        for hi in range(2):
            q = (qs[:, j] >> 4) if hi else (qs[:, j] & 0xF)
            d1 = (d * sc[:, 2 * j + hi].astype(np.float32)).astype(np.float32)
            m1 = (dm * mn[:, 2 * j + hi].astype(np.float32)).astype(np.float32)
            out[:, j, hi] = (d1[:, None] * q.astype(np.float32)).astype(np.float32) - m1[:, None]
    return out.reshape(-1)


def test_q4_k_both_scale_branches_against_gguf_restatement():
    rng = np.random.default_rng(10)
    blocks = rng.integers(0, 256, (300, 144), dtype=np.uint8)
    dvals = np.array([0x0001, 0x03FF, 0x0400, 0x3C00, 0x7BFF, 0x1234, 0x8400], np.uint16)
    blocks[:, 0:2] = dvals[np.arange(300) % 7].view(np.uint8).reshape(300, 2)
    blocks[:, 2:4] = dvals[(np.arange(300) + 3) % 7].view(np.uint8).reshape(300, 2)
    got = oracle.dequant(blocks, oracle.Q4_K, 300 * 256)
    assert np.array_equal(_bits(got), _bits(_q4k_gguf_layout(blocks)))


def test_q6_k_matches_reference_test_generator_and_kat():
    """resident.rs:712-738 generator bit-exact; quant.rs:2715-2737 scale-index KAT (Σ = 1920)."""
    blocks, deq = random_q6_k_blocks(100, WgpuLcg())
    assert np.array_equal(_bits(oracle.dequant(blocks, oracle.Q6_K, 100 * 256)), _bits(deq))
    blk = np.zeros(210, np.uint8)
    blk[:128], blk[128:192] = 0x11, 0xAA
    blk[192:208] = np.arange(16)
    blk[208:210] = np.array([np.float16(1.0)]).view(np.uint8)
    y = oracle.dequant(blk, oracle.Q6_K, 256)
    assert np.array_equal(y, np.repeat(np.arange(16, dtype=np.float32), 16)) and y.sum() == 1920.0


def test_q4_0_split_nibble_layout_and_exact_values():
    """tensor.rs:362-376 / gguf.rs:259-283 (the ggml split order): byte j of a block holds element j in its
    low nibble and element j + 16 in its high nibble, each q − 8, times d — exact in f32. Every byte value
    at every position under scales that include subnormal, negative and large d."""
    dvals = np.array([0x0001, 0x03FF, 0x3C00, 0xBC00, 0x7BFF, 0x2E66], np.uint16)
    for dv in dvals:
        d = float(np.array([dv], np.uint16).view(np.float16)[0])
        for j in range(16):
            blocks = np.zeros((256, 18), np.uint8)
            blocks[:, 0:2] = np.array([dv], np.uint16).view(np.uint8)
            blocks[:, 2:] = 0x88                              # every other element decodes to 0
            blocks[:, 2 + j] = np.arange(256, dtype=np.uint32).astype(np.uint8)
            y = oracle.dequant(blocks, oracle.Q4_0, 256 * 32).reshape(256, 32).astype(np.float64)
            v = np.arange(256)
            want = np.zeros((256, 32))
            want[:, j] = ((v & 0xF) - 8) * d
            want[:, j + 16] = ((v >> 4) - 8) * d
            assert np.array_equal(y, want), (hex(int(dv)), j)


def test_q5_k_reference_kat():
    """tensor.rs:800-830: d = 1, dmin = 0, sc = 1, m = 0 everywhere; qh[5] bit 0 and qh[0] bit 2 set, ql[3] = 2
    → element 3 is 2, elements 5 and 64 are 16 (the per-element high bit), every other element 0."""
    blk = np.zeros(176, np.uint8)
    blk[0:2] = np.array([np.float16(1.0)]).view(np.uint8)
    blk[2:4] = np.array([np.float16(0.0)]).view(np.uint8)
    blk[4:8] = 1
    blk[12:16] = 1
    blk[16 + 5] = 0b0000_0001
    blk[16 + 0] = 0b0000_0100
    blk[48 + 3] = 0x02
    y = oracle.dequant(blk, oracle.Q5_K, 256)
    want = np.zeros(256, np.float32)
    want[3], want[5], want[64] = 2.0, 16.0, 16.0
    assert np.array_equal(y, want)


def _q5k_f64(blocks: np.ndarray) -> np.ndarray:
    """The Q5_K values in float64: d·sc·(q + 16·h) and dmin·m are exact there, so rounding their difference once
    to f32 gives the reference's f32 result (whose products are exact and whose subtraction rounds once).
    Element 64c + 32·half + l: q = nibble `half` of ql[32c + l], h = bit 2c + half of qh[l], (sc, m) of
    sub-block 2c + half."""
    b = blocks.reshape(-1, 176)
    d = b[:, 0:2].copy().view(np.float16).astype(np.float64)[:, 0]
    dm = b[:, 2:4].copy().view(np.float16).astype(np.float64)[:, 0]
    s = b[:, 4:16].astype(np.int64)
    sc = np.concatenate([s[:, 0:4] & 63, (s[:, 8:12] & 0xF) | ((s[:, 0:4] >> 6) << 4)], axis=1)
    mn = np.concatenate([s[:, 4:8] & 63, (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)], axis=1)
    qh = b[:, 16:48].astype(np.int64)
    ql = b[:, 48:176].astype(np.int64).reshape(-1, 4, 32)
    out = np.empty((b.shape[0], 4, 2, 32))
    for c in range(4):
        for half in range(2):
            q = (ql[:, c] >> (4 * half)) & 0xF
            h = (qh >> (2 * c + half)) & 1
            sb = 2 * c + half
            out[:, c, half] = (d * sc[:, sb])[:, None] * (q + 16 * h) - (dm * mn[:, sb])[:, None]
    return out.reshape(-1).astype(np.float32)


def test_q5_k_exact_against_float64_and_every_bit_plane():
    rng = np.random.default_rng(13)
    blocks = rng.integers(0, 256, (300, 176), dtype=np.uint8)
    dvals = np.array([0x0001, 0x03FF, 0x0400, 0x3C00, 0x7BFF, 0x1234, 0x8400], np.uint16)
    blocks[:, 0:2] = dvals[np.arange(300) % 7].view(np.uint8).reshape(300, 2)
    blocks[:, 2:4] = dvals[(np.arange(300) + 3) % 7].view(np.uint8).reshape(300, 2)
    got = oracle.dequant(blocks, oracle.Q5_K, 300 * 256)
    assert np.array_equal(_bits(got), _bits(_q5k_f64(blocks)))
    # one qh bit at a time: bit p of qh[l] adds 16·d·sc to element 64·(p // 2) + 32·(p % 2) + l only
    base = np.zeros(176, np.uint8)
    base[0:2] = np.array([np.float16(1.0)]).view(np.uint8)
    base[4:8], base[12:16] = 1, 1                             # sc = 1, m = 0 for all eight sub-blocks
    for l in range(32):
        for p in range(8):
            blk = base.copy()
            blk[16 + l] = 1 << p
            y = oracle.dequant(blk, oracle.Q5_K, 256)
            assert np.flatnonzero(y).tolist() == [64 * (p // 2) + 32 * (p % 2) + l] and y.max() == 16.0


def test_embed_row_gather_matches_full_dequant():
    """common.rs:678-718: vocab 17 x 256, seed 0xABCD, ids [0, 7, 16, 3]; OOR id errors."""
    vocab, hidden = 17, 256
    data = gather_test_values(vocab, hidden)
    q8 = oracle.quantize_q8_0(data)
    ids = [0, 7, 16, 3]
    rng = np.random.default_rng(0xABCD)
    q4_0 = rng.integers(0, 256, (vocab * hidden // 32, 18), dtype=np.uint8)
    q4_0[:, 0:2] = np.frombuffer(rng.uniform(-0.05, 0.05, len(q4_0)).astype(np.float16).tobytes(),
                                 np.uint8).reshape(-1, 2)
    q5_k = rng.integers(0, 256, (vocab * hidden // 256, 176), dtype=np.uint8)
    q5_k[:, 0:4] = np.frombuffer(rng.uniform(0.001, 0.05, 2 * len(q5_k)).astype(np.float16).tobytes(),
                                 np.uint8).reshape(-1, 4)
    for dt, table, full in ((oracle.F32, data, data.reshape(-1)),
                            (oracle.F16, f16_bits(data), f16_bits(data).view(np.float16).astype(np.float32)),
                            (oracle.Q8_0, q8, oracle.dequant(q8, oracle.Q8_0, vocab * hidden)),
                            (oracle.Q4_0, q4_0, oracle.dequant(q4_0, oracle.Q4_0, vocab * hidden)),
                            (oracle.Q5_K, q5_k, oracle.dequant(q5_k, oracle.Q5_K, vocab * hidden))):
        got = oracle.embed_tokens(table, dt, vocab, hidden, ids)
        assert np.array_equal(_bits(got), _bits(full.reshape(vocab, hidden)[ids]))
    with pytest.raises(oracle.OracleError) as e:
        oracle.embed_tokens(data, oracle.F32, vocab, hidden, [vocab])
    assert e.value.status == oracle.ERANGE


def test_row_bytes_match_dtype_byte_count():
    """dtype.rs:136-145 byte_count for one row."""
    assert oracle.row_bytes(oracle.Q8_0, 896) == 952
    assert oracle.row_bytes(oracle.Q4_K, 4096) == 2304
    assert oracle.row_bytes(oracle.Q6_K, 4096) == 3360
    assert oracle.row_bytes(oracle.Q4_0, 896) == 504
    assert oracle.row_bytes(oracle.Q5_K, 4096) == 2816
    assert oracle.row_bytes(oracle.F16, 10) == 20
    assert oracle.row_bytes(oracle.Q8_0, 48) == 0   # not a whole number of blocks


def test_kv_append_q8_0_rows_are_quantized_blocks():
    """common.rs:449-508: each appended row of the quantized cache is quantize_f32_to_q8_0_block
    (common.rs:336-348) of its 32-element blocks — the quantizer pinned above against the wgpu tests'
    quantizer (resident.rs:506-524) — at byte (h · max_seq + position) · row_bytes; other rows untouched."""
    n_kv, seq, hd, max_seq, pos = 3, 5, 64, 12, 4
    src = WgpuLcg().take(n_kv * seq * hd).reshape(n_kv, seq, hd)
    row = hd // 32 * 34
    cache = np.full((n_kv, max_seq, row), 0xAB, np.uint8)
    oracle.kv_append(src, cache, oracle.Q8_0, n_kv, seq, hd, max_seq, pos)
    for h in range(n_kv):
        for s_ in range(seq):
            blocks, _ = quantize_q8_0_blocks(src[h, s_])
            assert np.array_equal(cache[h, pos + s_], blocks.reshape(-1))
    untouched = [p for p in range(max_seq) if not pos <= p < pos + seq]
    assert (cache[:, untouched] == 0xAB).all()


def test_transpose_heads_is_the_axis_permutation():
    """wgpu tests/resident.rs:956-982 (7 x 5 x 16, lcg): out[h][s][c] = x[s][h][c] and the round
    trip is the identity; numpy's axis permutation is the independent statement; half tensors
    move as raw 16-bit patterns (NaN payloads kept)."""
    x = WgpuLcg().take(7 * 5 * 16).reshape(7, 5, 16)
    t = oracle.transpose_heads(x, 7, 5, 16)
    assert np.array_equal(_bits(t), _bits(np.transpose(x, (1, 0, 2))))
    assert np.array_equal(_bits(oracle.transpose_heads(t, 5, 7, 16)), _bits(x))
    h = np.arange(3 * 4 * 6, dtype=np.uint16).reshape(3, 4, 6) | np.uint16(0x7C01)  # f16 NaN patterns
    assert np.array_equal(oracle.transpose_heads(h, 3, 4, 6), np.transpose(h, (1, 0, 2)))


@pytest.mark.parametrize("cache_dtype", [0, 1, 30])
def test_kv_append_is_a_slice_assignment(cache_dtype):
    """wgpu tests/resident.rs:339-415: a 3-token prefill then single-token decode appends into a
    [2, 16, 64] cache; the cache equals numpy slice assignment of the RNE-rounded values
    (f16 via numpy's float16, bf16 via torch) and nothing else is written; pos + seq > max_seq
    is an error."""
    n_kv, hd, max_seq, steps = 2, 64, 16, 6
    nxt = WgpuLcg()
    dt = np.float32 if cache_dtype == 0 else np.uint16
    cache = np.zeros((n_kv, max_seq, hd), dt)
    want = np.zeros((n_kv, max_seq, hd), np.float32)
    chunk = nxt.take(n_kv * 3 * hd).reshape(n_kv, 3, hd)
    oracle.kv_append(chunk, cache, cache_dtype, n_kv, 3, hd, max_seq, 0)
    want[:, 0:3] = chunk
    for t in range(3, steps):
        knew = nxt.take(n_kv * hd).reshape(n_kv, 1, hd)
        oracle.kv_append(knew, cache, cache_dtype, n_kv, 1, hd, max_seq, t)
        want[:, t:t + 1] = knew
    if cache_dtype == 0:
        assert np.array_equal(_bits(cache), _bits(want))
    elif cache_dtype == 1:
        assert np.array_equal(cache, want.astype(np.float16).view(np.uint16))
    else:
        assert np.array_equal(cache, torch.from_numpy(want).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16))
    assert (cache[:, steps:] == 0).all()
    with pytest.raises(oracle.OracleError):
        oracle.kv_append(np.zeros((n_kv, 2, hd), np.float32), cache, cache_dtype, n_kv, 2, hd, max_seq, 15)


def test_kv_cache_update_reference_kat():
    """crates/sapient-models/tests/inference_test.rs:10-61: an f32 cache [1, 2, 4, 2]; one token, then
    two more at seq 1; views of length 1 and 3; the cache holds 1,3,4 / 2,5,6 and zeros past them."""
    cache = np.zeros((2, 4, 2), np.float32)
    assert oracle.kv_cache_update(np.array([1, 1, 2, 2], np.float32), cache, oracle.F32, 2, 1, 2, 4, 0) == 1
    k2 = np.array([3, 3, 4, 4, 5, 5, 6, 6], np.float32)
    assert oracle.kv_cache_update(k2, cache, oracle.F32, 2, 2, 2, 4, 1) == 3
    assert np.array_equal(cache[0].reshape(-1), [1, 1, 3, 3, 4, 4, 0, 0])
    assert np.array_equal(cache[1].reshape(-1), [2, 2, 5, 5, 6, 6, 0, 0])


def _window_model(old_rows: np.ndarray, new_rows: np.ndarray, max_seq: int) -> np.ndarray:
    """The sliding window stated as what it keeps: the last min(len, max_seq) rows of the valid
    rows followed by the new ones (independent of the shift-then-insert loop of common.rs)."""
    both = np.concatenate([old_rows, new_rows], axis=1)
    return both[:, max(0, both.shape[1] - max_seq):]


@pytest.mark.parametrize("cache_dtype", [0, 1, 30, 8])
@pytest.mark.parametrize("max_seq,cur_len,seq", [(8, 0, 3), (8, 5, 3), (8, 8, 1), (8, 7, 3), (8, 6, 8), (8, 0, 8),
                                                 (8, 8, 8), (5, 5, 4), (16, 16, 1), (16, 3, 15), (1, 1, 1)])
def test_kv_cache_update_is_a_sliding_window(cache_dtype, max_seq, cur_len, seq):
    """common.rs:355-434 / :449-508 (f32, f16, bf16 and Q8_0 caches): after the update the first
    new_len = min(cur_len + seq, max_seq) rows of every head are the last new_len rows of
    (old valid rows, new rows converted to the cache type); rows past new_len are untouched."""
    n_kv, hd = 3, 64
    rng = np.random.default_rng(max_seq * 100 + cur_len * 10 + seq + cache_dtype)
    if cache_dtype == oracle.Q8_0:
        row = hd // 32 * 34
        cache = rng.integers(0, 256, (n_kv, max_seq, row), dtype=np.uint8)
    elif cache_dtype == 0:
        row = hd
        cache = rng.standard_normal((n_kv, max_seq, row), dtype=np.float32)
    else:
        row = hd
        cache = rng.integers(0, 1 << 16, (n_kv, max_seq, row), dtype=np.uint16)
    before = cache.copy()
    src = rng.standard_normal((n_kv, seq, hd), dtype=np.float32) * 3
    if cache_dtype == oracle.Q8_0:
        new = np.stack([np.stack([quantize_q8_0_blocks(src[h, s_])[0].reshape(-1) for s_ in range(seq)])
                        for h in range(n_kv)])
    elif cache_dtype == 0:
        new = src
    elif cache_dtype == 1:
        new = src.astype(np.float16).view(np.uint16)
    else:
        new = torch.from_numpy(src).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    n = oracle.kv_cache_update(src, cache, cache_dtype, n_kv, seq, hd, max_seq, cur_len)
    assert n == min(cur_len + seq, max_seq)
    want = _window_model(before[:, :cur_len], new, max_seq)
    assert np.array_equal(_bits(cache[:, :n]) if cache_dtype == 0 else cache[:, :n],
                          _bits(want) if cache_dtype == 0 else want)
    assert np.array_equal(cache[:, n:], before[:, n:])


def test_kv_cache_update_errors():
    """seq > max_seq is the reference's bail (common.rs:378-379); cur_len > max_seq has no valid
    meaning (its subtraction would underflow); nothing is written in either case."""
    cache = np.zeros((2, 4, 2), np.float32)
    with pytest.raises(oracle.OracleError):
        oracle.kv_cache_update(np.zeros(2 * 5 * 2, np.float32), cache, oracle.F32, 2, 5, 2, 4, 0)
    with pytest.raises(oracle.OracleError):
        oracle.kv_cache_update(np.zeros(2 * 1 * 2, np.float32), cache, oracle.F32, 2, 1, 2, 4, 5)
    assert (cache == 0).all()
