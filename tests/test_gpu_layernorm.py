"""GPU parity: LayerNorm against the oracle.

Reference: crates/sapient-backends/cpu/src/kernels/layernorm.rs:17-69 (layer_norm over
the last axis, weight and bias each optional), reached through LlmBackend::layer_norm
(crates/sapient-models/src/forward/backend.rs:73-79 → common.rs:575-577).

Tolerance. The kernel sums Σx and Σ(x − mean)² in a different order than the
reference's serial folds; every other step rounds alike. A serial f32 fold of n
values moves the mean by about 2^-24·√n·(|mean| + σ) and the variance alike, so
y = normed·w + b may differ by
    |Δ| ≤ |w| · (1 + |normed|) · 8 · 2^-24 · √n · (|mean| + σ) / σ  +  2^-22 · |y|
(8 is the margin over the random-walk estimate). Half outputs: ≤ 1 ulp against
the f32 oracle rounded to nearest-even, or within that bound plus half an ulp
of the output format.
"""
import numpy as np
import pytest
import torch

from helpers import assert_ulp16, check_layer_norm, max_rel, narrow_bits, to_np, ulp_diff16, widen
from refvec import WgpuLcg

import sapient_amd.ops as ops

pytestmark = pytest.mark.gpu
DTYPES = [torch.float32, torch.float16, torch.bfloat16]
IDS = lambda d: str(d).split(".")[-1]


def _gen(shape, seed, dev, mean=0.0, std=1.0, dtype=torch.float32):
    g = torch.Generator(device=dev).manual_seed(seed)
    return (torch.randn(shape, generator=g, device=dev) * std + mean).to(dtype)


def test_layer_norm_matches_wgpu_test_vectors(dev, orc):
    """wgpu tests/resident.rs:860-886: 7 x 1536, lcg, x·3, w = 0.5 + |next()|, b = next()·0.1,
    eps 1e-5; the reference test's own bound is 1e-4 absolute."""
    rows, dim = 7, 1536
    nxt = WgpuLcg()
    x = (nxt.take(rows * dim) * np.float32(3.0)).reshape(rows, dim)
    w = np.float32(0.5) + np.abs(nxt.take(dim))
    b = nxt.take(dim) * np.float32(0.1)
    print(f"case layer_norm wgpu-vectors {rows}x{dim}", flush=True)
    out = ops.layer_norm(torch.from_numpy(x).to(dev), torch.from_numpy(w).to(dev), torch.from_numpy(b).to(dev), 1e-5)
    ref = orc.layer_norm(x, w, b, 1e-5)
    check_layer_norm(out, ref, x, w, b, orc, "wgpu vectors")
    x64 = x.astype(np.float64)
    mu, var = x64.mean(axis=1, keepdims=True), x64.var(axis=1, keepdims=True)
    assert np.abs(to_np(out) - ((x64 - mu) / np.sqrt(var + 1e-5) * w + b)).max() < 1e-4


def _run(dev, orc, dtype, rows, dim, mode, wbt, od):
    print(f"case layer_norm {dtype} {rows}x{dim} {mode} wb={wbt} out={od}", flush=True)
    x = _gen((rows, dim), 2000 + dim, dev, 0.7, 2.0, dtype)
    w = _gen((dim,), 5, dev, 1.0, 0.3, wbt) if "w" in mode else None
    b = _gen((dim,), 6, dev, 0.0, 0.2, wbt) if mode in ("wb", "b") else None
    out = ops.layer_norm(x, w, b, 1e-5, out_dtype=od)
    x32 = widen(x, orc)
    w32 = None if w is None else widen(w, orc)
    b32 = None if b is None else widen(b, orc)
    ref = orc.layer_norm(x32, w32, b32, 1e-5)
    check_layer_norm(out, ref, x32, w32, b32, orc, f"layer_norm {dtype} {rows}x{dim} {mode}")


@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
@pytest.mark.parametrize("rows,dim", [(1, 384), (7, 1536), (3, 1280), (512, 768), (7, 64), (2, 4), (33, 4096),
                                      (4, 8192), (3, 8200), (2, 16384), (3, 100), (1, 1)])
@pytest.mark.parametrize("mode", ["wb", "w", "b", "none"])
def test_layer_norm_shapes(dev, orc, dtype, rows, dim, mode):
    """Weight / bias in x's type, output in x's type (the half-resident layout)."""
    _run(dev, orc, dtype, rows, dim, mode, dtype, dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=IDS)
@pytest.mark.parametrize("rows,dim", [(7, 1536), (3, 8200), (3, 100)])
@pytest.mark.parametrize("wbmode,outmode", [("f32", "same"), ("f32", "f32"), ("same", "f32")])
def test_layer_norm_mixed_types(dev, orc, dtype, rows, dim, wbmode, outmode):
    """Half x with f32 weight / bias and / or f32 output (the reference's f32 result)."""
    _run(dev, orc, dtype, rows, dim, "wb", torch.float32 if wbmode == "f32" else dtype,
         torch.float32 if outmode == "f32" else dtype)


@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
@pytest.mark.parametrize("rows,dim", [(16384, 4096), (1500, 1280)])
def test_layer_norm_full(dev, orc, dtype, rows, dim):
    """16384 x 4096 (the benchmark's Llama-3-8B width) and 1500 x 1280 (Whisper-large encoder)."""
    print(f"case layer_norm full {dtype} {rows}x{dim}", flush=True)
    x = _gen((rows, dim), 71, dev, 0.5, 1.5, dtype)
    w = _gen((dim,), 72, dev, 1.0, 0.2)
    b = _gen((dim,), 73, dev, 0.0, 0.1)
    out = ops.layer_norm(x, w, b, 1e-5)
    torch.cuda.synchronize()
    x32 = widen(x, orc)
    ref = orc.layer_norm(x32, to_np(w), to_np(b), 1e-5)
    check_layer_norm(out, ref, x32, to_np(w), to_np(b), orc, f"layer_norm full {dtype}")


@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
@pytest.mark.parametrize("dim", [4096, 100, 64, 4])
@pytest.mark.parametrize("mode", ["none", "w", "b", "wb"])
def test_layer_norm_signed_zero_bit_exact(dev, orc, dtype, dim, mode):
    """Rows of (k, -k) pairs (k = 1, 2, 3), one -0 and one +0, shuffled: every sum the kernel forms is an
    exact integer in any order, so its mean (+0), variance and outputs equal the oracle's bit for bit. The
    -0 element centres to -0 - (+0) = -0, and without a bias the reference writes -0·w
    (layernorm.rs:17-69): an absent bias enters the kernel as -0, the identity of +, which keeps that
    sign (+0 would not). Weights of both signs; 4096 takes the row-looping shape, 100 (halves) the
    one-element kernel."""
    rng = np.random.default_rng(dim * 8 + len(mode))
    pairs = [np.float32(1 + i % 3) for i in range((dim - 2) // 2)]
    proto = np.array([v for k in pairs for v in (k, -k)] + [-0.0, 0.0], np.float32)
    x32 = np.stack([rng.permutation(proto) for _ in range(3)]).astype(np.float32)
    x = torch.from_numpy(x32).to(dev).to(dtype)
    w = torch.from_numpy(rng.normal(0.0, 1.0, dim).astype(np.float32)).to(dev).to(dtype) if "w" in mode else None
    b = torch.from_numpy(rng.normal(0.0, 0.2, dim).astype(np.float32)).to(dev).to(dtype) if "b" in mode else None
    print(f"case layer_norm signed zero {dtype} 3x{dim} {mode}", flush=True)
    out = ops.layer_norm(x, w, b, 1e-5)
    ref = orc.layer_norm(widen(x, orc), None if w is None else widen(w, orc), None if b is None else widen(b, orc), 1e-5)
    if dtype == torch.float32:
        got, want = to_np(out).view(np.uint32), ref.view(np.uint32)
    else:
        got, want = to_np(out), narrow_bits(ref, dtype, orc)
    assert np.array_equal(got, want), f"{int((got != want).sum())} of {got.size} outputs differ in bits"
    if mode == "none":
        neg0 = np.signbit(x32) & (x32 == 0)
        assert np.all(np.signbit(ref[neg0])) and np.all(ref[neg0] == 0)


def test_layer_norm_unit_property(dev):
    """Size-independent check at the full shape: with no weight / bias and eps = 0
    every output row has mean 0 and variance 1 (to f32 rounding)."""
    x = _gen((16384, 4096), 81, dev, 5.0, 3.0)
    out = ops.layer_norm(x, None, None, 0.0).double()
    assert out.mean(dim=1).abs().max().item() < 1e-5
    assert (out.var(dim=1, unbiased=False) - 1).abs().max().item() < 1e-5


def test_layer_norm_kat(dev):
    """layernorm.rs:113-123: [[1, 2], [3, 4]] → [[-1, 1], [-1, 1]] within 1e-4."""
    x = torch.tensor([[1.0, 2.0], [3.0, 4.0]], device=dev)
    out = ops.layer_norm(x, None, None, 1e-5).cpu().numpy()
    assert np.abs(out - np.array([[-1, 1], [-1, 1]])).max() < 1e-4


def test_layer_norm_unaligned_views_take_generic_path(dev, orc):
    base = _gen((4 * 768 + 1,), 91, dev, 1.0, 2.0)
    x = base[1:].view(4, 768)
    out = torch.empty(4 * 768 + 1, device=dev)[1:].view(4, 768)
    w = _gen((768,), 92, dev, 1.0, 0.1)
    b = _gen((768,), 93, dev, 0.0, 0.1)
    ops.layer_norm(x, w, b, 1e-5, out=out)
    ref = orc.layer_norm(to_np(x), to_np(w), to_np(b), 1e-5)
    check_layer_norm(out, ref, to_np(x), to_np(w), to_np(b), orc, "unaligned")


def test_layer_norm_rejects_bad_arguments(dev):
    from sapient_amd._lib import EINVAL, lib
    L = lib()
    x = torch.zeros(4, 8, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    p = x.data_ptr()
    assert L.sph_layer_norm(p, 5, None, None, 0, p, 0, 4, 8, 1e-5, s) == EINVAL          # x dtype
    assert L.sph_layer_norm(None, 0, None, None, 0, p, 0, 4, 8, 1e-5, s) == EINVAL       # null x
    assert L.sph_layer_norm(p, 1, p, None, 30, p, 1, 4, 8, 1e-5, s) == EINVAL           # weight dtype
    assert L.sph_layer_norm(p, 1, None, None, 0, p, 30, 4, 8, 1e-5, s) == EINVAL        # out dtype
    assert L.sph_layer_norm(p, 0, None, None, 0, p, 0, -1, 8, 1e-5, s) == EINVAL        # negative rows
    with pytest.raises(ValueError, match="does not match last dim"):
        ops.layer_norm(x, torch.ones(7, device=dev), None, 1e-5)
