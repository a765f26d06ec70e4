"""GPU parity over randomly drawn shapes, storage offsets and dtypes, against the oracle.

The fixed-shape tests pin each op at the configurations and at chosen edges; this
sweep draws cases the fixed ones do not name (seeded, every case printed before it
runs) so that the launch-shape choices — vector widths, waves per row, row looping,
one- or two-vector element launches, folded RoPE grids and head groups, element-
aligned fallbacks — meet odd dimensions, small and large row counts and every
pointer alignment an element offset produces:

  rms_norm / add_rms_norm   layernorm.rs:75-106, llama.rs:508→515
  layer_norm                layernorm.rs:17-69
  silu, swiglu, gelu_tanh,  elementwise.rs:15-69, :120-143, :163-174
  gelu_erf, add, mul
  add_bias                  common.rs:556-569
  rope (both layouts,       rope.rs:18-62, :83-136; gguf_weights.rs:111-115
  partial, scaled, q + k)
  transpose_heads           resident.rs:420-458
  kv_append                 resident.rs:645-711
  fused decode step         wgpu_engine.rs:397-432, :525-573 (bias + RoPE + append,
                            heads-major and token-major)

Bars, as in the fixed tests: RMSNorm f32 outputs ≤ 1e-5 relative and half outputs
≤ 1 ulp of the oracle's f32 result rounded to nearest-even (the kernel's Σx² is
summed in another order); LayerNorm within the fixed tests' summation-order bound
(helpers.layer_norm_bound); the fused residual, the element-wise ops, the bias,
RoPE and the layout moves bit for bit.
"""
import numpy as np
import pytest
import torch

from helpers import (assert_bits16_equal, assert_bits_equal, assert_ulp16, check_layer_norm, max_rel, narrow_bits,
                     to_np, widen)

import sapient_amd.ops as ops
from sapient_amd._lib import BF16, F16, F32

pytestmark = pytest.mark.gpu
DTYPES = [torch.float32, torch.float16, torch.bfloat16]
CODE = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}
CASES = 100


def _name(d):
    return str(d).split(".")[-1]


def _dim(rng, top):
    """A last dimension: tiny, small odd, near a multiple of 4 / 8 / 64 / 1024, or large."""
    kind = rng.integers(0, 5)
    if kind == 0:
        return int(rng.integers(1, 17))
    if kind == 1:
        return int(rng.integers(17, 700)) | 1
    if kind == 2:
        m = int(rng.choice([4, 8, 64]))
        return max(1, m * int(rng.integers(1, 200)) + int(rng.integers(-3, 4)))
    if kind == 3:
        return max(1, 1024 * int(rng.integers(1, 17)) + int(rng.integers(-2, 3)))
    return int(rng.integers(700, top))


def _tensor(shape, dtype, dev, seed, offset, std=1.0, mean=0.0):
    """A tensor of `shape` placed `offset` elements into a larger allocation (element-aligned only)."""
    n = int(np.prod(shape)) if len(shape) else 1
    g = torch.Generator(device=dev).manual_seed(seed)
    raw = (torch.randn(n + offset, generator=g, device=dev) * std + mean).to(dtype)
    return raw[offset:offset + n].view(shape)


def _same_bits(out: torch.Tensor, ref32: np.ndarray, orc, what: str):
    if out.dtype == torch.float32:
        assert_bits_equal(to_np(out), ref32, what)
    else:
        assert_bits16_equal(to_np(out).reshape(-1), narrow_bits(ref32, out.dtype, orc).reshape(-1), what)


def _norm_close(out: torch.Tensor, ref32: np.ndarray, orc, what: str):
    if out.dtype == torch.float32:
        r = max_rel(to_np(out), ref32)
        assert r <= 1e-5, f"{what}: max rel err {r:.3e}"
    else:
        assert_ulp16(to_np(out), narrow_bits(ref32, out.dtype, orc), out.dtype, 1, what)


@pytest.mark.parametrize("case", range(CASES))
def test_norms_random_shapes(dev, orc, case):
    rng = np.random.default_rng(1000 + case)
    dtype = DTYPES[case % 3]
    rows = int(rng.choice([1, 2, 3, 7, 16, 33, 100, 257]))
    dim = _dim(rng, 20000)
    while rows * dim > 600_000:
        rows = max(1, rows // 2)
    wmode = rng.choice(["none", "f32", "same"])
    omode = rng.choice(["same", "f32"])
    offs = [int(o) for o in rng.integers(0, 4, 4)]
    eps = float(rng.choice([1e-6, 1e-5]))
    print(f"case norms {case}: {_name(dtype)} {rows}x{dim} w={wmode} out={omode} offsets={offs}", flush=True)
    x = _tensor((rows, dim), dtype, dev, 3 * case + 1, offs[0])
    r = _tensor((rows, dim), dtype, dev, 3 * case + 2, offs[1])
    wdt = torch.float32 if wmode == "f32" or dtype == torch.float32 else dtype
    w = None if wmode == "none" else _tensor((dim,), wdt, dev, 3 * case + 3, offs[2], 0.1, 1.0)
    odt = torch.float32 if omode == "f32" else dtype
    x32, r32 = widen(x, orc), widen(r, orc)
    w32 = None if w is None else widen(w, orc)
    out = ops.rms_norm(x, w, eps, out_dtype=odt)
    _norm_close(out, orc.rms_norm(x32, w32, eps), orc, f"rms_norm case {case}")
    # out of place first (the residual must come back unchanged), then in place; the sum buffer is
    # as aligned as the residual in odd cases (then the launch is the in-place one's, bit for bit)
    so = offs[1] if case % 2 else (offs[1] + 1) % 4
    sm = torch.empty(rows * dim + so, dtype=dtype, device=dev)[so:].view(rows, dim)
    y_to = torch.empty(rows * dim + offs[3], dtype=odt, device=dev)[offs[3]:].view(rows, dim)
    r_before = r.clone()
    ops.add_rms_norm(x, r, w, eps, out=y_to, sum_out=sm)
    assert np.array_equal(to_np(r).view(np.uint8), to_np(r_before).view(np.uint8)), f"residual kept, case {case}"
    y = torch.empty(rows * dim + offs[3], dtype=odt, device=dev)[offs[3]:].view(rows, dim)
    ops.add_rms_norm(x, r, w, eps, out=y)
    ref_y, ref_r = orc.add_rms_norm(x32, r32, w32, eps)
    _same_bits(r, ref_r, orc, f"add_rms_norm residual case {case}")
    _norm_close(y, ref_y, orc, f"add_rms_norm case {case}")
    _same_bits(sm, ref_r, orc, f"add_rms_norm_to sum case {case}")
    _norm_close(y_to, ref_y, orc, f"add_rms_norm_to case {case}")
    if so == offs[1]:
        assert np.array_equal(to_np(y_to).view(np.uint8), to_np(y).view(np.uint8)), f"add_rms_norm_to output case {case}"


@pytest.mark.parametrize("case", range(CASES))
def test_layer_norm_random_shapes(dev, orc, case):
    rng = np.random.default_rng(1500 + case)
    dtype = DTYPES[case % 3]
    rows = int(rng.choice([1, 2, 3, 7, 16, 33, 100, 257]))
    dim = _dim(rng, 20000)
    while rows * dim > 600_000:
        rows = max(1, rows // 2)
    mode = rng.choice(["wb", "w", "b", "none"])
    wbdt = torch.float32 if rng.integers(0, 2) or dtype == torch.float32 else dtype
    odt = torch.float32 if rng.integers(0, 2) else dtype
    offs = [int(o) for o in rng.integers(0, 4, 3)]
    print(f"case layer_norm {case}: {_name(dtype)} {rows}x{dim} {mode} wb {_name(wbdt)} out {_name(odt)} "
          f"offsets={offs}", flush=True)
    x = _tensor((rows, dim), dtype, dev, 3 * case + 1, offs[0], 1.5, 0.5)
    w = _tensor((dim,), wbdt, dev, 3 * case + 2, offs[1], 0.2, 1.0) if "w" in mode else None
    b = _tensor((dim,), wbdt, dev, 3 * case + 3, offs[2], 0.1) if "b" in mode else None
    x32 = widen(x, orc)
    w32 = None if w is None else widen(w, orc)
    b32 = None if b is None else widen(b, orc)
    out = ops.layer_norm(x, w, b, 1e-5, out_dtype=odt)
    check_layer_norm(out, orc.layer_norm(x32, w32, b32, 1e-5), x32, w32, b32, orc, f"layer_norm case {case}")


@pytest.mark.parametrize("case", range(CASES))
def test_elementwise_random_shapes(dev, orc, case):
    rng = np.random.default_rng(2000 + case)
    dtype = DTYPES[case % 3]
    kind = rng.integers(0, 3)
    n = int(rng.integers(1, 40)) if kind == 0 else int(rng.integers(40, 70_000)) if kind == 1 else \
        int(rng.integers(70_000, 2_000_000))
    offs = [int(o) for o in rng.integers(0, 4, 3)]
    print(f"case elementwise {case}: {_name(dtype)} n={n} offsets={offs}", flush=True)
    a = _tensor((n,), dtype, dev, 5 * case + 1, offs[0], 2.5)
    b = _tensor((n,), dtype, dev, 5 * case + 2, offs[1], 2.5)
    a32, b32 = widen(a, orc), widen(b, orc)
    out = torch.empty(n + offs[2], dtype=dtype, device=dev)[offs[2]:]
    for fn, ref in ((ops.silu, orc.silu(a32)), (ops.gelu_tanh, orc.gelu(a32)), (ops.gelu_erf, orc.gelu_erf(a32))):
        _same_bits(fn(a, out=out), ref, orc, f"{fn.__name__} case {case}")
    _same_bits(ops.swiglu(a, b, out=out), orc.swiglu(a32, b32), orc, f"swiglu case {case}")
    # add / mul, sometimes with a length-1 operand on either side (elementwise.rs:41-48)
    side = rng.integers(0, 3)
    s = _tensor((1,), dtype, dev, 5 * case + 3, 0)
    lhs, rhs = (a, b) if side == 0 else (a, s) if side == 1 else (s, b)
    l32, r32 = widen(lhs, orc), widen(rhs, orc)
    _same_bits(ops.add(lhs, rhs, out=out), orc.add(l32, r32), orc, f"add case {case} side {side}")
    _same_bits(ops.mul(lhs, rhs, out=out), orc.mul(l32, r32), orc, f"mul case {case} side {side}")


@pytest.mark.parametrize("case", range(CASES))
def test_add_bias_random_shapes(dev, orc, case):
    rng = np.random.default_rng(3000 + case)
    dtype = DTYPES[case % 3]
    n = _dim(rng, 12000)
    rows = int(rng.integers(1, max(2, 400_000 // n)))
    bdt = torch.float32 if rng.integers(0, 2) or dtype == torch.float32 else dtype
    offs = [int(o) for o in rng.integers(0, 4, 2)]
    print(f"case add_bias {case}: {_name(dtype)} {rows}x{n} bias {_name(bdt)} offsets={offs}", flush=True)
    y = _tensor((rows, n), dtype, dev, 2 * case + 1, offs[0])
    bias = _tensor((n,), bdt, dev, 2 * case + 2, offs[1], 0.5)
    _same_bits(ops.add_bias(y, bias), orc.add_bias_last_dim(widen(y, orc), widen(bias, orc)), orc,
               f"add_bias case {case}")


@pytest.mark.parametrize("case", range(CASES))
def test_rope_random_shapes(dev, orc, case):
    rng = np.random.default_rng(4000 + case)
    dtype = DTYPES[case % 3]
    interleaved = bool(case % 2)
    half = int(rng.choice([1, 2, 3, 4, 6, 8, 16, 20, 32, 48, 64, 128, int(rng.integers(1, 257))]))
    D = 2 * half
    rd = D if rng.integers(0, 3) else 2 * int(rng.integers(1, half + 1))
    if rng.integers(0, 4) == 0 and D < 1000:
        D += 2 * int(rng.integers(1, 8))  # channels past the rotary ones pass through
    B = int(rng.integers(1, 3))
    S = int(rng.choice([1, 2, 3, 5, 17, 64, 255, 256, 257, 700]))
    Hq = int(rng.integers(1, 20))
    Hk = int(rng.integers(0, 5))
    while B * (Hq + Hk) * S * D > 1_500_000 and S > 1:
        S //= 2
    base = float(rng.choice([1e4, 5e5, 1e6]))
    pos_scale = float(rng.choice([1.0, 1.0, 4.0, 0.25]))
    positions = [int(p) for p in rng.integers(0, 40_000, S)]
    offs = [int(o) for o in rng.integers(0, 4, 2)]
    print(f"case rope {case}: {_name(dtype)} {'il' if interleaved else 'neox'} B{B} Hq{Hq} Hk{Hk} S{S} D{D} "
          f"rd{rd} base {base} scale {pos_scale} offsets={offs}", flush=True)
    q = _tensor((B, Hq, S, D), dtype, dev, 2 * case + 1, offs[0])
    k = _tensor((B, Hk, S, D), dtype, dev, 2 * case + 2, offs[1]) if Hk else None
    q32 = widen(q, orc).reshape(B, Hq, S, D)
    k32 = widen(k, orc).reshape(B, Hk, S, D) if Hk else None
    ops.rope_(q, k, torch.tensor(positions, dtype=torch.int32, device=dev), base, rotary_dim=rd,
              pos_scale=pos_scale, interleaved=interleaved)
    _same_bits(q, orc.apply_rope_partial_scaled(q32, positions, base, rd, pos_scale, interleaved), orc,
               f"rope q case {case}")
    if Hk:
        _same_bits(k, orc.apply_rope_partial_scaled(k32, positions, base, rd, pos_scale, interleaved), orc,
                   f"rope k case {case}")


@pytest.mark.parametrize("case", range(CASES))
def test_layout_moves_random_shapes(dev, orc, case):
    rng = np.random.default_rng(5000 + case)
    dtype = DTYPES[case % 3]
    cdt = DTYPES[int(rng.integers(0, 3))]
    outer, inner = int(rng.integers(1, 40)), int(rng.integers(1, 300))
    hd = int(rng.choice([1, 2, 3, 6, 12, 32, 64, 80, 128, 256]))
    max_seq = inner + int(rng.integers(0, 50))
    pos = int(rng.integers(0, max_seq - inner + 1))
    offs = [int(o) for o in rng.integers(0, 4, 2)]
    print(f"case layout {case}: {_name(dtype)} -> cache {_name(cdt)} [{outer}, {inner}, {hd}] max_seq {max_seq} "
          f"pos {pos} offsets={offs}", flush=True)
    x = _tensor((outer, inner, hd), dtype, dev, 2 * case + 1, offs[0])
    t = ops.transpose_heads(x)
    want = orc.transpose_heads(to_np(x), outer, inner, hd)
    assert np.array_equal(to_np(t).view(want.dtype), want), f"transpose_heads case {case}"
    cache = _tensor((outer, max_seq, hd), cdt, dev, 2 * case + 2, offs[1])
    ref = to_np(cache).copy()
    ops.kv_append(x, cache, pos)
    orc.kv_append(widen(x, orc), ref, CODE[cdt], outer, inner, hd, max_seq, pos)
    got = to_np(cache)
    assert np.array_equal(got.view(np.uint32) if got.dtype == np.float32 else got,
                          ref.view(np.uint32) if ref.dtype == np.float32 else ref), f"kv_append case {case}"


def _round_to(x32: np.ndarray, dtype, orc) -> np.ndarray:
    """f32 values rounded to `dtype` (nearest-even) and widened back: a store in that type."""
    if dtype == torch.float32:
        return x32.astype(np.float32)
    bits = narrow_bits(x32, dtype, orc)
    return orc.f16_bits_to_f32(bits) if dtype == torch.float16 else orc.bf16_bits_to_f32(bits)


@pytest.mark.parametrize("case", range(CASES))
def test_fused_decode_step_random_shapes(dev, orc, case):
    """sph_rope_kv_append (heads-major, q in place) and sph_rope_kv_append_tokens (token-major in,
    q out heads-major) against the oracle's unfused sequence, wgpu_engine.rs:397-432 / :525-573:
    bias added in f32 and stored in the activation type, RoPE over the full head (stored in the
    activation type again for k), then each token's k and v rows appended at its own position in
    the cache type. Positions are a random subset of the cache rows, in random order."""
    rng = np.random.default_rng(6000 + case)
    dtype = DTYPES[case % 3]
    cdt = DTYPES[int(rng.integers(0, 3))]
    bmode = rng.choice(["none", "f32", "same"])
    bdt = torch.float32 if bmode == "f32" or dtype == torch.float32 else dtype
    token_major = bool(rng.integers(0, 2))
    interleaved = bool(rng.integers(0, 2))
    Hq, Hkv = int(rng.integers(1, 24)), int(rng.integers(1, 9))
    D = 8 * int(rng.choice([1, 2, 3, 5, 8, 10, 12, 16, 32]))
    S = int(rng.choice([1, 2, 3, 4, 5, 9, 64, 300]))
    max_seq = S + int(rng.integers(0, 300))
    base = float(rng.choice([1e4, 5e5, 1e6]))
    positions = np.sort(rng.permutation(max_seq)[:S]).astype(np.int32)
    if rng.integers(0, 2):
        positions = rng.permutation(positions).astype(np.int32)
    print(f"case fused {case}: {_name(dtype)} cache {_name(cdt)} bias {bmode} {'tokens' if token_major else 'heads'} "
          f"{'il' if interleaved else 'neox'} Hq{Hq} Hkv{Hkv} S{S} D{D} max_seq {max_seq}", flush=True)
    shp = (lambda H: (S, H, D)) if token_major else (lambda H: (H, S, D))
    q = _tensor(shp(Hq), dtype, dev, 7 * case + 1, 0)
    k = _tensor(shp(Hkv), dtype, dev, 7 * case + 2, 0)
    v = _tensor(shp(Hkv), dtype, dev, 7 * case + 3, 0)
    biases = [None if bmode == "none" else _tensor((H * D,), bdt, dev, 7 * case + 4 + i, 0, 0.1)
              for i, H in enumerate((Hq, Hkv, Hkv))]
    kc = _tensor((Hkv, max_seq, D), cdt, dev, 7 * case + 7, 0)
    vc = _tensor((Hkv, max_seq, D), cdt, dev, 7 * case + 8, 0)
    kref, vref = to_np(kc).copy(), to_np(vc).copy()

    def heads_major(t, H):  # exact f32 values, [H, S, D]
        a = widen(t, orc).reshape(shp(H))
        return np.ascontiguousarray(a.transpose(1, 0, 2) if token_major else a)

    def biased(a, b, H):
        return a if b is None else _round_to(a + widen(b, orc).reshape(H, 1, D), dtype, orc)

    q32 = biased(heads_major(q, Hq), biases[0], Hq)
    k32 = biased(heads_major(k, Hkv), biases[1], Hkv)
    v32 = biased(heads_major(v, Hkv), biases[2], Hkv)
    pos_t = torch.from_numpy(positions).to(dev)
    if token_major:
        q_out = ops.rope_kv_append_tokens(q, k, v, pos_t, base, kc, vc, interleaved=interleaved,
                                          bq=biases[0], bk=biases[1], bv=biases[2])
    else:
        ops.rope_kv_append(q, k, v, pos_t, base, kc, vc, interleaved=interleaved,
                           bq=biases[0], bk=biases[1], bv=biases[2])
        q_out = q
    rope = lambda a: orc.apply_rope_partial_scaled(a[None], positions, base, D, 1.0, interleaved)[0]
    _same_bits(q_out, rope(q32), orc, f"fused q case {case}")
    kr = _round_to(rope(k32), dtype, orc)
    for s, p in enumerate(positions.tolist()):
        orc.kv_append(np.ascontiguousarray(kr[:, s:s + 1]), kref, CODE[cdt], Hkv, 1, D, max_seq, p)
        orc.kv_append(np.ascontiguousarray(v32[:, s:s + 1]), vref, CODE[cdt], Hkv, 1, D, max_seq, p)
    for got, want, what in ((to_np(kc), kref, "k cache"), (to_np(vc), vref, "v cache")):
        eq = got.view(np.uint32) == want.view(np.uint32) if got.dtype == np.float32 else got == want
        assert eq.all(), f"fused {what} case {case}: {int((~eq).sum())} elements differ"
