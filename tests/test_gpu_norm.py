"""GPU parity: RMSNorm and fused residual-add + RMSNorm against the oracle.

Reference: crates/sapient-backends/cpu/src/kernels/layernorm.rs:75-106 (rms_norm),
crates/sapient-models/src/forward/llama.rs:508→515 (add then rms_norm).

Tolerances (stated by the op set's parity contract):
  f32 outputs  ≤ 1e-5 relative, element-wise (the kernel sums Σx² in a different
               order than the reference's serial fold; everything else rounds alike)
  f16 / bf16   ≤ 1 ulp of the output format against the f32 oracle rounded to
               nearest-even
  residual     bit-exact (one IEEE add, then the same rounding)
"""
import numpy as np
import pytest
import torch

from helpers import assert_ulp16, assert_bits16_equal, assert_bits_equal, max_rel, narrow_bits, to_np, ulp_diff16, widen
from refvec import WgpuLcg

import sapient_amd.ops as ops

pytestmark = pytest.mark.gpu
RTOL = 1e-5
DTYPES = [torch.float32, torch.float16, torch.bfloat16]


def _gen(shape, seed, dev, mean=0.0, std=1.0, dtype=torch.float32):
    g = torch.Generator(device=dev).manual_seed(seed)
    return (torch.randn(shape, generator=g, device=dev) * std + mean).to(dtype)


def _check_out(out: torch.Tensor, ref32: np.ndarray, orc, what: str):
    if out.dtype == torch.float32:
        r = max_rel(to_np(out), ref32)
        assert r <= RTOL, f"{what}: max rel err {r:.3e} > {RTOL}"
    else:
        assert_ulp16(to_np(out), narrow_bits(ref32, out.dtype, orc), out.dtype, 1, what)


def test_rms_norm_matches_wgpu_test_vectors(dev, orc):
    """resident.rs:28-59: 5 x 1536, LCG seed 0x12345678, w = 0.5 + |next()|, eps 1e-5."""
    rows, dim = 5, 1536
    nxt = WgpuLcg(0x12345678)
    x = nxt.take(rows * dim).reshape(rows, dim)
    w = np.float32(0.5) + np.abs(nxt.take(dim))
    print(f"case rms_norm wgpu-vectors {rows}x{dim}", flush=True)
    out = ops.rms_norm(torch.from_numpy(x).to(dev), torch.from_numpy(w).to(dev), 1e-5)
    got = to_np(out)
    ref = orc.rms_norm(x, w, 1e-5)
    assert max_rel(got, ref) <= RTOL
    # the reference test's own bound and restatement (abs 1e-4)
    ms = (x.astype(np.float64) ** 2).mean(axis=1, keepdims=True)
    want = x / np.sqrt(ms + 1e-5) * w
    assert np.abs(got - want).max() < 1e-4


# (input dtype, weight dtype mode, output dtype mode): every distinct combination (for f32 input, "same"
# weight / output is the f32 case itself).
_RMS_MODES = [pytest.param(dt, wm, om, id=f"{str(dt).split('.')[-1]}-w{wm}-out{om}")
              for dt in DTYPES for wm in ("f32", "same", "none") for om in ("same", "f32")
              if not (dt == torch.float32 and (wm == "same" or om == "f32"))]


@pytest.mark.parametrize("rows,dim", [(1, 896), (3, 896), (512, 896), (7, 64), (2, 4), (5, 1536), (33, 4096),
                                      (4, 8192), (3, 8200), (2, 16384), (3, 100), (1, 1)])
@pytest.mark.parametrize("dtype,wmode,outmode", _RMS_MODES)
def test_rms_norm_shapes(dev, orc, dtype, rows, dim, wmode, outmode):
    print(f"case rms_norm {dtype} {rows}x{dim} w={wmode} out={outmode}", flush=True)
    x = _gen((rows, dim), 1000 + dim, dev, dtype=dtype)
    w = None if wmode == "none" else _gen((dim,), 7, dev, 1.0, 0.1, torch.float32 if wmode == "f32" else dtype)
    eps = 1e-6
    out = ops.rms_norm(x, w, eps, out_dtype=torch.float32 if outmode == "f32" else dtype)
    ref = orc.rms_norm(widen(x, orc), None if w is None else widen(w, orc), eps)
    _check_out(out, ref, orc, f"rms_norm {dtype} {rows}x{dim}")


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("rows,dim", [(1, 896), (512, 896), (33, 4096), (4, 8192), (3, 8200), (2, 12288), (2, 16384),
                                      (600, 1024), (3, 100)])
def test_add_rms_norm_shapes(dev, orc, dtype, rows, dim):
    """Widths that take each launch shape: the row-looping one (up to 4096 f32 / 8192 half
    elements), one block per row, twice the values per lane past 16 waves, and the generic kernel."""
    print(f"case add_rms_norm {dtype} {rows}x{dim}", flush=True)
    x = _gen((rows, dim), 11 + dim, dev, dtype=dtype)
    r = _gen((rows, dim), 13 + dim, dev, dtype=dtype)
    w = _gen((dim,), 17, dev, 1.0, 0.1)
    x32, r32 = widen(x, orc), widen(r, orc)
    out, r_new = ops.add_rms_norm(x, r, w, 1e-5)
    ref, ref_r = orc.add_rms_norm(x32, r32, widen(w, orc), 1e-5)
    _check_out(out, ref, orc, f"add_rms_norm {dtype} {rows}x{dim}")
    if dtype == torch.float32:
        assert_bits_equal(to_np(r_new), ref_r, "updated residual")
    else:
        assert_bits16_equal(to_np(r_new), narrow_bits(ref_r, dtype, orc), "updated residual")


def _same_bits(a: torch.Tensor, b: torch.Tensor) -> bool:
    return torch.equal(a.contiguous().view(torch.uint8), b.contiguous().view(torch.uint8))


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("rows,dim", [(1, 896), (512, 896), (33, 4096), (2, 12288), (2, 16384), (3, 100),
                                      (16384, 4096)])
def test_add_rms_norm_to_equals_in_place(dev, orc, dtype, rows, dim):
    """The out-of-place form (sph_add_rms_norm_to): the residual is left as it was, and the sum and
    the normed rows are the in-place form's bit for bit, across the launch shapes and at the full
    16384 x 4096 shape (the sum also against the oracle)."""
    print(f"case add_rms_norm_to {dtype} {rows}x{dim}", flush=True)
    x = _gen((rows, dim), 51 + dim, dev, dtype=dtype)
    r = _gen((rows, dim), 53 + dim, dev, dtype=dtype)
    w = _gen((dim,), 57, dev, 1.0, 0.1)
    r_before = r.clone()
    out_to, s = ops.add_rms_norm(x, r, w, 1e-5, sum_out=torch.empty_like(r))
    torch.cuda.synchronize()
    assert _same_bits(r, r_before), "residual left as it was"
    out_in, r_in = ops.add_rms_norm(x, r.clone(), w, 1e-5)
    torch.cuda.synchronize()
    assert _same_bits(s, r_in), "sum equals the in-place residual"
    assert _same_bits(out_to, out_in), "normed rows equal the in-place form's"
    if rows * dim <= 1 << 20:
        ref_r = orc.add_rms_norm(widen(x, orc), widen(r_before, orc), widen(w, orc), 1e-5)[1]
        if dtype == torch.float32:
            assert_bits_equal(to_np(s), ref_r, "sum")
        else:
            assert_bits16_equal(to_np(s), narrow_bits(ref_r, dtype, orc), "sum")


def test_add_rms_norm_to_unaligned_and_half_outputs(dev, orc):
    """The generic kernel (a 4-byte offset view) and an f16 output with an f16 weight, out of place."""
    base = _gen((4 * 896 + 1,), 61, dev)
    x = base[1:].view(4, 896)
    r = _gen((4, 896), 62, dev)
    s = torch.empty(4 * 896 + 1, device=dev)[1:].view(4, 896)
    w = _gen((896,), 63, dev, 1.0, 0.1)
    out, _ = ops.add_rms_norm(x, r, w, 1e-6, sum_out=s)
    ref, ref_r = orc.add_rms_norm(to_np(x), to_np(r), to_np(w), 1e-6)
    assert_bits_equal(to_np(s), ref_r, "unaligned sum")
    assert max_rel(to_np(out), ref) <= RTOL
    xh, rh, wh = (_gen((8, 1024), 64 + i, dev, dtype=torch.float16) for i in range(3))
    outh, sh = ops.add_rms_norm(xh, rh, wh[0], 1e-5, sum_out=torch.empty_like(rh))
    refh, refh_r = orc.add_rms_norm(widen(xh, orc), widen(rh, orc), widen(wh[0], orc), 1e-5)
    assert_bits16_equal(to_np(sh), narrow_bits(refh_r, torch.float16, orc), "f16 sum")
    _check_out(outh, refh, orc, "f16 out of place")


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
def test_add_rms_norm_llama3_8b_full(dev, orc, dtype):
    """Fused add + RMSNorm at Llama-3-8B width, 16384 x 4096, eps 1e-5, the full benchmark shape."""
    rows, dim = 16384, 4096
    print(f"case add_rms_norm full {dtype} {rows}x{dim}", flush=True)
    x = _gen((rows, dim), 21, dev, dtype=dtype)
    r = _gen((rows, dim), 22, dev, dtype=dtype)
    w = _gen((dim,), 23, dev, 1.0, 0.1)
    x32, r32 = widen(x, orc), widen(r, orc)
    out, r_new = ops.add_rms_norm(x, r, w, 1e-5)
    torch.cuda.synchronize()
    ref, ref_r = orc.add_rms_norm(x32, r32, widen(w, orc), 1e-5)
    _check_out(out, ref, orc, f"add_rms_norm full {dtype}")
    if dtype == torch.float32:
        assert_bits_equal(to_np(r_new), ref_r, "updated residual")
    else:
        assert_bits16_equal(to_np(r_new), narrow_bits(ref_r, dtype, orc), "updated residual")


def test_rms_norm_unit_rms_property(dev):
    """Size-independent check at the full shape: with w = 1 and eps = 0 every
    output row has mean square 1 (to f32 rounding)."""
    x = _gen((16384, 4096), 31, dev, std=3.0)
    out = ops.rms_norm(x, None, 0.0)
    ms = (out.double() ** 2).mean(dim=1)
    assert torch.allclose(ms, torch.ones_like(ms), rtol=0, atol=2e-6)


def test_rms_norm_kat(dev):
    """layernorm.rs:126-149: x = [3, 4], w = 1, eps = 0 → [3, 4] / sqrt(12.5)."""
    x = torch.tensor([[3.0, 4.0]], device=dev)
    out = ops.rms_norm(x, torch.ones(2, device=dev), 0.0).cpu()
    e0 = np.float32(3.0) / np.sqrt(np.float32(12.5))
    e1 = np.float32(4.0) / np.sqrt(np.float32(12.5))
    assert abs(out[0, 0].item() - e0) < 1e-5 and abs(out[0, 1].item() - e1) < 1e-5


def test_rms_norm_unaligned_views_take_generic_path(dev, orc):
    """Pointers that are not 16-byte aligned must still be correct (generic kernel)."""
    base = _gen((4 * 896 + 1,), 41, dev)
    x = base[1:].view(4, 896)  # 4-byte offset
    out = torch.empty(4 * 896 + 1, device=dev)[1:].view(4, 896)
    w = _gen((896,), 42, dev, 1.0, 0.1)
    ops.rms_norm(x, w, 1e-6, out=out)
    ref = orc.rms_norm(to_np(x), to_np(w), 1e-6)
    assert max_rel(to_np(out), ref) <= RTOL


def test_rms_norm_rejects_bad_arguments(dev):
    from sapient_amd._lib import EINVAL, lib
    L = lib()
    x = torch.zeros(4, 8, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    assert L.sph_rms_norm(x.data_ptr(), 5, None, 0, x.data_ptr(), 0, 4, 8, 1e-5, s) == EINVAL  # dtype
    assert L.sph_rms_norm(None, 0, None, 0, x.data_ptr(), 0, 4, 8, 1e-5, s) == EINVAL        # null x
    assert L.sph_add_rms_norm(x.data_ptr(), x.data_ptr(), 0, None, 0, x.data_ptr(), 0, 4, 8, 1e-5, s) == EINVAL
    r, y, t = torch.zeros(4, 8, device=dev), torch.zeros(4, 8, device=dev), torch.zeros(4, 8, device=dev)
    to = L.sph_add_rms_norm_to
    assert to(x.data_ptr(), r.data_ptr(), x.data_ptr(), 0, None, 0, y.data_ptr(), 0, 4, 8, 1e-5, s) == EINVAL  # sum = x
    assert to(x.data_ptr(), r.data_ptr(), t.data_ptr(), 0, None, 0, t.data_ptr(), 0, 4, 8, 1e-5, s) == EINVAL  # out = sum
    assert to(x.data_ptr(), r.data_ptr(), None, 0, None, 0, y.data_ptr(), 0, 4, 8, 1e-5, s) == EINVAL  # null sum
    assert to(x.data_ptr(), r.data_ptr(), t.data_ptr(), 7, None, 0, y.data_ptr(), 0, 4, 8, 1e-5, s) == EINVAL  # dtype
    # sum = residual is the in-place form
    x1 = torch.ones(4, 8, device=dev)
    assert to(x1.data_ptr(), r.data_ptr(), r.data_ptr(), 0, None, 0, y.data_ptr(), 0, 4, 8, 1e-5, s) == 0
    torch.cuda.synchronize()
    assert torch.equal(r, x1) and torch.allclose(y, torch.ones_like(y))
    assert L.sph_rms_norm(x.data_ptr(), 1, x.data_ptr(), 0, x.data_ptr(), 30, 4, 8, 1e-5, s) == EINVAL  # out dtype
