"""GPU: the op set where a 32-bit element index would wrap, and past the
per-launch chunks the host code splits work into (2^22 rows for the row
kernels, 2^24 tokens for the embedding gather).

Tensors of 2^31 + a few elements (4 GiB of f16). Where the op has an exact
identity (x · 1 = x, a transpose) every element is checked on the device;
otherwise the first and last elements or rows — those past index 2^31 are the
ones a wrapped index would lose or overwrite — are checked against the oracle
at the op's own bar (bit-exact, or ≤ 1 ulp for the half RMSNorm).
"""
import numpy as np
import pytest
import torch

from helpers import narrow_bits, to_np, ulp_diff16, widen

import sapient_amd.ops as ops
from sapient_amd._lib import Q8_0

pytestmark = pytest.mark.gpu
BIG = (1 << 31) + 40


@pytest.fixture(autouse=True)
def _release():
    yield
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def _ends(t: torch.Tensor, k: int) -> torch.Tensor:
    f = t.reshape(-1)
    return torch.cat([f[:k], f[-k:]])


def _randn(n, dev, dtype, seed, scale=1.0):
    g = torch.Generator(device=dev).manual_seed(seed)
    return (torch.randn(n, generator=g, device=dev) * scale).to(dtype)


def test_mul_by_one_beyond_2g_elements(dev):
    a = _randn(BIG, dev, torch.float16, 1)
    print("case mul f16 2^31+40 elements", flush=True)
    out = ops.mul(a, torch.ones(1, device=dev, dtype=torch.float16))
    assert torch.equal(out, a)  # x · 1 = x exactly, all 2^31 + 40 elements compared on the device


def test_swiglu_and_gelu_beyond_2g_elements(dev, orc):
    g = _randn(BIG, dev, torch.float16, 2, 2.0)
    u = _randn(BIG, dev, torch.float16, 3, 2.0)
    k = 1 << 16
    gn, un = widen(_ends(g, k), orc), widen(_ends(u, k), orc)
    print("case swiglu f16 2^31+40 elements", flush=True)
    s = ops.swiglu(g, u)
    assert np.array_equal(to_np(_ends(s, k)), narrow_bits(orc.swiglu(gn, un), torch.float16, orc))
    del s, u
    print("case gelu_tanh f16 2^31+40 elements", flush=True)
    y = ops.gelu_tanh(g)
    assert np.array_equal(to_np(_ends(y, k)), narrow_bits(orc.gelu(gn), torch.float16, orc))


def test_rms_norm_half_beyond_2g_elements(dev, orc):
    rows, dim = (1 << 20) + 3, 2048  # 2^31 + 6144 elements
    x = _randn(rows * dim, dev, torch.float16, 4).view(rows, dim)
    w = _randn(dim, dev, torch.float32, 5, 0.1) + 1
    print(f"case rms_norm f16 {rows}x{dim}", flush=True)
    y = ops.rms_norm(x, w, 1e-5)
    for sl in (slice(0, 8), slice(rows - 8, rows)):
        want = narrow_bits(orc.rms_norm(widen(x[sl], orc).reshape(-1, dim), to_np(w), 1e-5), torch.float16, orc)
        assert ulp_diff16(to_np(y[sl]).reshape(-1), want.reshape(-1), torch.float16).max() <= 1


@pytest.mark.parametrize("dim", [8, 7], ids=["vector", "generic"])
def test_rms_norm_rows_past_the_launch_chunk(dev, orc, dim):
    """2^22 + 5 rows: two launches of the row kernel (vector path, and the generic path for dim 7)."""
    rows = (1 << 22) + 5
    x = _randn(rows * dim, dev, torch.float32, 6).view(rows, dim)
    w = _randn(dim, dev, torch.float32, 7, 0.1) + 1
    print(f"case rms_norm f32 {rows}x{dim}", flush=True)
    got = to_np(ops.rms_norm(x, w, 1e-6))
    want = orc.rms_norm(to_np(x), to_np(w), 1e-6)
    assert np.max(np.abs(got - want) / np.maximum(np.abs(want), 1e-30)) <= 1e-5


def test_add_bias_beyond_2g_elements(dev, orc):
    rows, n = (1 << 19) + 1, 4096  # 2^31 + 4096 elements
    y = _randn(rows * n, dev, torch.float16, 8).view(rows, n)
    b = _randn(n, dev, torch.float16, 9)
    print(f"case add_bias f16 {rows}x{n}", flush=True)
    out = ops.add_bias(y, b)
    for sl in (slice(0, 4), slice(rows - 4, rows)):
        want = narrow_bits(orc.add_bias_last_dim(widen(y[sl], orc).reshape(-1, n), widen(b, orc)), torch.float16,
                           orc)
        assert np.array_equal(to_np(out[sl]), want.reshape(-1, n))


def test_transpose_heads_beyond_2g_elements(dev):
    outer, inner, hd = (1 << 20) + 1, 16, 128  # 2^31 + 2048 elements
    x = _randn(outer * inner * hd, dev, torch.float16, 10).view(outer, inner, hd)
    print(f"case transpose_heads f16 {outer}x{inner}x{hd}", flush=True)
    out = ops.transpose_heads(x)
    assert torch.equal(out, x.transpose(0, 1).contiguous())  # every element, on the device


def test_rope_beyond_2g_elements(dev, orc):
    H, S, D = 8, (1 << 21) + 1, 128  # 2^31 + 1024 elements
    q = _randn(H * S * D, dev, torch.float16, 11).view(1, H, S, D)
    pos = torch.arange(S, dtype=torch.int32, device=dev)
    ends = [q[:, :, :4].clone(), q[:, :, -4:].clone()]
    print(f"case rope f16 1x{H}x{S}x{D}", flush=True)
    ops.rope_(q, None, pos, 5e5)
    for got, before, p in ((q[:, :, :4], ends[0], np.arange(4)), (q[:, :, -4:], ends[1], np.arange(S - 4, S))):
        want = orc.apply_rope(widen(before, orc).reshape(1, H, 4, D), p, 5e5)
        assert np.array_equal(to_np(got).reshape(-1), narrow_bits(want, torch.float16, orc).reshape(-1))


def test_embed_past_the_token_chunk_and_2g_outputs(dev, orc):
    """2^24 + 100 tokens (two launches) of a Q8_0 table, 2^31 + 12800 f32 outputs."""
    vocab, hidden, n = 1000, 128, (1 << 24) + 100
    rng = np.random.default_rng(12)
    nb = vocab * hidden // 32
    table = rng.integers(0, 256, nb * 34, dtype=np.uint8).reshape(nb, 34)
    table[:, 0:2] = np.frombuffer(rng.uniform(0.001, 0.05, nb).astype(np.float16).tobytes(), np.uint8).reshape(nb, 2)
    ids = torch.randint(0, vocab, (n,), dtype=torch.int32, device=dev)
    print(f"case embed q8_0 {n} ids x {hidden}", flush=True)
    out = ops.embed(torch.from_numpy(table.reshape(-1)).to(dev), Q8_0, vocab, hidden, ids)
    for lo, hi in ((0, 64), ((1 << 24) - 32, (1 << 24) + 32), (n - 64, n)):
        got = to_np(out[lo:hi])
        want = orc.embed_tokens(table.reshape(-1), Q8_0, vocab, hidden, to_np(ids[lo:hi]).view(np.uint32))
        assert np.array_equal(got.view(np.uint32), want.reshape(hi - lo, hidden).view(np.uint32))


@pytest.mark.parametrize("q8", [False, True], ids=["f16", "q8_0"])
def test_kv_cache_update_past_the_head_chunk(dev, orc, q8):
    """65535 + 100 heads: the window kernels split heads across launches (grid y holds at most 65535);
    both forms of the update (in place and into a second cache) match the oracle on every row."""
    n_kv, hd, max_seq, cur = 65535 + 100, 32, 8, 8
    code = Q8_0 if q8 else 1
    row = hd // 32 * 34 if q8 else hd
    g = torch.Generator(device=dev).manual_seed(21)
    src = torch.randn(n_kv, 1, hd, generator=g, device=dev)
    if q8:
        cache = torch.randint(0, 256, (n_kv, max_seq, row), generator=g, device=dev, dtype=torch.int32).to(torch.uint8)
    else:
        cache = torch.randn(n_kv, max_seq, hd, generator=g, device=dev).half()
    before = to_np(cache).copy()
    want = before.copy()
    assert orc.kv_cache_update(to_np(src), want, code, n_kv, 1, hd, max_seq, cur) == max_seq
    print(f"case kv_cache_update_into {n_kv} heads {'q8_0' if q8 else 'f16'}", flush=True)
    out = torch.zeros_like(cache)
    assert ops.kv_cache_update_into(src, cache, out, cur) == max_seq
    assert np.array_equal(to_np(out).view(np.uint8), want.view(np.uint8))
    assert np.array_equal(to_np(cache).view(np.uint8), before.view(np.uint8))
    print(f"case kv_cache_update in place {n_kv} heads {'q8_0' if q8 else 'f16'}", flush=True)
    assert ops.kv_cache_update(src, cache, cur) == max_seq
    assert np.array_equal(to_np(cache).view(np.uint8), want.view(np.uint8))
