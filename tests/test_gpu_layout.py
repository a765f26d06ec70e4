"""GPU parity: the device-resident decode helpers against the oracle.

Reference: crates/sapient-backends/wgpu/src/resident.rs:420-458 (transpose_heads)
and :645-711 (kv_append), with their tests tests/resident.rs:339-415 and :956-982.

Both are moves: bit-exact. Same-type moves keep every bit pattern (NaN payloads
included); f32 → f16 / bf16 cache writes round to nearest-even, bit-exact
against the oracle's narrowing.
"""
import numpy as np
import pytest
import torch

from helpers import assert_bits16_equal, assert_bits_equal, to_np, widen
from refvec import WgpuLcg

import sapient_amd.ops as ops

pytestmark = pytest.mark.gpu
DTYPES = [torch.float32, torch.float16, torch.bfloat16]
IDS = lambda d: str(d).split(".")[-1]
CODE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 30}


def _gen(shape, seed, dev, dtype=torch.float32):
    g = torch.Generator(device=dev).manual_seed(seed)
    return torch.randn(shape, generator=g, device=dev).to(dtype)


def _same(got: torch.Tensor, want: np.ndarray, what: str):
    if got.dtype == torch.float32:
        assert_bits_equal(to_np(got), want, what)
    else:
        assert_bits16_equal(to_np(got), want, what)


def test_transpose_heads_matches_wgpu_test(dev, orc):
    """tests/resident.rs:956-982: [7, 5, 16] → [5, 7, 16] and back is the identity."""
    x = WgpuLcg().take(7 * 5 * 16).reshape(7, 5, 16)
    print("case transpose wgpu-vectors", flush=True)
    t = ops.transpose_heads(torch.from_numpy(x).to(dev))
    assert_bits_equal(to_np(t), orc.transpose_heads(x, 7, 5, 16), "forward")
    back = ops.transpose_heads(t)
    assert_bits_equal(to_np(back), x, "round trip")


@pytest.mark.parametrize("dtype", DTYPES, ids=IDS)
@pytest.mark.parametrize("outer,inner,hd", [(8192, 32, 128), (1, 32, 128), (512, 14, 64), (7, 5, 16), (3, 4, 6),
                                            (5, 3, 9), (1, 1, 1), (33, 8, 80)])
def test_transpose_heads_shapes(dev, orc, dtype, outer, inner, hd):
    print(f"case transpose {dtype} {outer}x{inner}x{hd}", flush=True)
    x = _gen((outer, inner, hd), outer * 31 + hd, dev, dtype)
    got = ops.transpose_heads(x)
    _same(got, orc.transpose_heads(to_np(x), outer, inner, hd), f"transpose {dtype}")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16], ids=IDS)
def test_transpose_heads_keeps_every_half_pattern(dev, orc, dtype):
    """All 65536 16-bit patterns (NaN payloads and signalling NaNs included) move unchanged."""
    bits = torch.arange(0, 65536, dtype=torch.int32).to(torch.int16).view(dtype).reshape(64, 8, 128).to(dev)
    got = ops.transpose_heads(bits)
    assert np.array_equal(to_np(got), np.transpose(to_np(bits), (1, 0, 2)))


def test_transpose_heads_unaligned_views_take_scalar_path(dev, orc):
    base = _gen((4 * 6 * 32 + 1,), 5, dev)
    x = base[1:].view(4, 6, 32)
    out = torch.empty(4 * 6 * 32 + 1, device=dev)[1:].view(6, 4, 32)
    ops.transpose_heads(x, out=out)
    assert_bits_equal(to_np(out), orc.transpose_heads(to_np(x), 4, 6, 32), "unaligned")


@pytest.mark.parametrize("cdtype", DTYPES, ids=IDS)
def test_kv_append_matches_wgpu_test_sequence(dev, orc, cdtype):
    """tests/resident.rs:339-415: n_kv 2, head_dim 64, max_seq 16; a 3-token prefill append
    then three single-token appends; the cache equals the oracle's bit for bit and positions
    past the last append are untouched."""
    n_kv, hd, max_seq, steps = 2, 64, 16, 6
    nxt = WgpuLcg()
    sentinel = 0x7E7E if cdtype != torch.float32 else 0x7E7E7E7E
    cache = torch.full((n_kv, max_seq, hd), sentinel, dtype=torch.int32 if cdtype == torch.float32 else torch.int16,
                       device=dev).view(cdtype)
    ref = to_np(cache).copy()
    chunk = nxt.take(n_kv * 3 * hd).reshape(n_kv, 3, hd)
    print(f"case kv_append sequence {cdtype}", flush=True)
    ops.kv_append(torch.from_numpy(chunk).to(dev), cache, 0)
    orc.kv_append(chunk, ref, CODE[cdtype], n_kv, 3, hd, max_seq, 0)
    for t in range(3, steps):
        knew = nxt.take(n_kv * hd).reshape(n_kv, 1, hd)
        ops.kv_append(torch.from_numpy(knew).to(dev), cache, t)
        orc.kv_append(knew, ref, CODE[cdtype], n_kv, 1, hd, max_seq, t)
    _same(cache, ref, f"kv cache {cdtype}")


# Every (source, cache) dtype pair at the small shapes (an f32 <-> half pair moves 8 elements per thread
# at hd 64 and 128, 4 at hd 12; hd 6 and 1 take the one-element path); the large prefill runs f32 sources
# into every cache type and half sources into f16.
_KV_CASES = [pytest.param(sd, cd, *shape, id=f"{IDS(sd)}-{IDS(cd)}-{'x'.join(map(str, shape))}")
             for sd in DTYPES for cd in DTYPES
             for shape in [(8, 8192, 128, 8192, 0), (8, 1, 128, 8192, 8191), (2, 5, 64, 40, 17), (2, 3, 12, 9, 2),
                           (3, 4, 6, 10, 6), (1, 1, 1, 1, 0)]
             if not (shape[1] == 8192 and sd != torch.float32 and cd != torch.float16)]


@pytest.mark.parametrize("sdtype,cdtype,n_kv,seq,hd,max_seq,pos", _KV_CASES)
def test_kv_append_shapes(dev, orc, sdtype, cdtype, n_kv, seq, hd, max_seq, pos):
    print(f"case kv_append {sdtype}->{cdtype} {n_kv}x{seq}x{hd} max {max_seq} pos {pos}", flush=True)
    src = _gen((n_kv, seq, hd), seq + hd, dev, sdtype)
    cache = _gen((n_kv, max_seq, hd), 99, dev, cdtype)
    ref = to_np(cache).copy()
    ops.kv_append(src, cache, pos)
    orc.kv_append(widen(src, orc), ref, CODE[cdtype], n_kv, seq, hd, max_seq, pos)
    _same(cache, ref, f"kv_append {sdtype}->{cdtype}")


def test_kv_append_rejects_out_of_range(dev):
    from sapient_amd._lib import EINVAL, ERANGE, SapientHipError, lib
    cache = torch.zeros(2, 8, 16, device=dev)
    before = cache.clone()
    with pytest.raises(SapientHipError):
        ops.kv_append(torch.ones(2, 3, 16, device=dev), cache, 6)
    assert torch.equal(cache, before)
    L = lib()
    s = torch.cuda.current_stream().cuda_stream
    p = cache.data_ptr()
    assert L.sph_kv_append(p, 0, p, 0, 2, 3, 16, 8, 6, s) == ERANGE
    assert L.sph_kv_append(p, 0, p, 0, 2, 1, 16, 8, 8, s) == ERANGE
    assert L.sph_kv_append(p, 0, p, 0, 2, 1, 16, 8, -1, s) == EINVAL
    assert L.sph_kv_append(p, 8, p, 0, 2, 1, 16, 8, 0, s) == EINVAL       # src dtype
    assert L.sph_transpose_heads(p, p, 0, 2, 8, 16, s) == EINVAL            # out aliases x
    assert L.sph_transpose_heads(p, None, 0, 2, 8, 16, s) == EINVAL


@pytest.mark.parametrize("sdtype", [torch.float32, torch.float16, torch.bfloat16], ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("n_kv,seq,hd,max_seq,pos", [(2, 1, 64, 16, 5), (8, 37, 128, 64, 20), (4, 512, 64, 600, 0)])
def test_kv_append_q8_0_cache(dev, orc, sdtype, n_kv, seq, hd, max_seq, pos):
    """The quantized KV cache (update_kv_cache_q8, common.rs:449-508): new rows quantized block by block on
    append, bit-exact with the oracle's quantizer; rows outside pos .. pos + seq untouched. The source mixes
    ordinary values with all-zero blocks, huge and tiny magnitudes, ties of v / scale at .5, and NaN / inf."""
    g = torch.Generator(device=dev).manual_seed(n_kv * 1000 + seq)
    src = torch.randn(n_kv, seq, hd, generator=g, device=dev) * 3
    flat = src.view(-1, 32)
    nb = flat.shape[0]
    flat[0::7] = 0.0                                                     # all-zero blocks
    flat[1::7] *= 1e6                                                    # scale overflows f16 (inf d)
    flat[2::7] *= 1e-30                                                  # subnormal scale
    flat[3::7] = torch.arange(32, device=dev, dtype=torch.float32) - 15.5  # v / scale lands on .5 ties
    if nb > 5:
        flat[5, 3] = float("nan")
        flat[5, 4] = float("inf")
    src = src.to(sdtype)
    row = hd // 32 * 34
    cache = torch.randint(0, 256, (n_kv, max_seq, row), generator=g, device=dev, dtype=torch.int32).to(torch.uint8)
    before = to_np(cache).copy()
    print(f"case kv_append q8_0 {sdtype} {n_kv}x{seq}x{hd} -> {max_seq} @ {pos}", flush=True)
    ops.kv_append(src, cache, pos)
    want = before.copy()
    orc.kv_append(widen(src, orc).reshape(n_kv, seq, hd), want, orc.Q8_0, n_kv, seq, hd, max_seq, pos)
    assert np.array_equal(to_np(cache), want)


def test_kv_append_q8_0_rejects_bad_shapes(dev):
    from sapient_amd._lib import EINVAL, ERANGE, Q8_0, lib
    src = torch.zeros(2, 3, 48, device=dev)
    cache = torch.zeros(2, 8, 64, dtype=torch.uint8, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    assert lib().sph_kv_append(src.data_ptr(), 0, cache.data_ptr(), Q8_0, 2, 3, 48, 8, 0, s) == EINVAL  # 48 % 32
    src = torch.zeros(2, 3, 64, device=dev)
    assert lib().sph_kv_append(src.data_ptr(), 0, cache.data_ptr(), Q8_0, 2, 3, 64, 8, 6, s) == ERANGE  # 6 + 3 > 8


# Sliding-window cache update (common.rs:355-434, :449-508): (n_kv, hd, max_seq, cur_len, seq). Covers no shift,
# a decode step on a full cache, a prefill chunk that slides, seq == max_seq (nothing kept), Llama-3-8B's
# 8 x 8192 x 128 cache at full length, and row widths that take each access width of the shift kernel
# (16-byte units, 8 (Q8_0 at hd 128: 136-byte rows), 4, 2 (hd 1 in f16, Q8_0 at hd 32: 34-byte rows)).
_UPD_CASES = [(2, 64, 16, 5, 3), (2, 64, 16, 16, 1), (3, 64, 16, 12, 7), (2, 64, 16, 9, 16), (2, 64, 16, 16, 16),
              (8, 128, 8192, 8192, 1), (8, 128, 8192, 8000, 512), (5, 3, 40, 40, 2), (4, 1, 33, 30, 5),
              (1, 128, 4096, 4095, 3), (11, 64, 100, 100, 1)]


@pytest.mark.parametrize("cdtype", [torch.float32, torch.float16, torch.bfloat16], ids=IDS)
@pytest.mark.parametrize("n_kv,hd,max_seq,cur_len,seq", _UPD_CASES)
def test_kv_cache_update_matches_oracle(dev, orc, cdtype, n_kv, hd, max_seq, cur_len, seq):
    """update_kv_cache on the device: the shift moves rows bit for bit, the new rows are converted as
    kv_append converts them, and the returned length is the reference view's; bit-exact with the oracle
    over the whole cache (rows past the new length untouched)."""
    print(f"case kv_cache_update {cdtype} {n_kv}x{hd} max {max_seq} cur {cur_len} seq {seq}", flush=True)
    src = _gen((n_kv, seq, hd), seq * 7 + hd, dev)
    cache = _gen((n_kv, max_seq, hd), 17 + hd, dev, cdtype)
    ref = to_np(cache).copy()
    n = ops.kv_cache_update(src, cache, cur_len)
    want_n = orc.kv_cache_update(to_np(src), ref, CODE[cdtype], n_kv, seq, hd, max_seq, cur_len)
    assert n == want_n == min(cur_len + seq, max_seq)
    _same(cache, ref, f"kv_cache_update {cdtype}")


@pytest.mark.parametrize("n_kv,hd,max_seq,cur_len,seq", [(2, 64, 16, 16, 1), (3, 32, 24, 20, 9), (8, 128, 512, 512, 1),
                                                         (2, 128, 64, 40, 64), (2, 64, 16, 3, 4)])
def test_kv_cache_update_q8_0(dev, orc, n_kv, hd, max_seq, cur_len, seq):
    """The quantized cache (update_kv_cache_q8): 34-byte blocks moved by the shift as raw bytes, new rows
    quantized on append; bit-exact with the oracle."""
    print(f"case kv_cache_update q8_0 {n_kv}x{hd} max {max_seq} cur {cur_len} seq {seq}", flush=True)
    g = torch.Generator(device=dev).manual_seed(max_seq + cur_len)
    src = torch.randn(n_kv, seq, hd, generator=g, device=dev) * 3
    row = hd // 32 * 34
    cache = torch.randint(0, 256, (n_kv, max_seq, row), generator=g, device=dev, dtype=torch.int32).to(torch.uint8)
    ref = to_np(cache).copy()
    n = ops.kv_cache_update(src, cache, cur_len)
    assert n == orc.kv_cache_update(to_np(src), ref, orc.Q8_0, n_kv, seq, hd, max_seq, cur_len)
    assert np.array_equal(to_np(cache), ref)


def test_kv_cache_update_decode_sequence(dev, orc):
    """Thirty decode steps past a full f16 cache (the window slides one row per step), each step checked
    against the oracle's cache after the same steps."""
    n_kv, hd, max_seq = 4, 64, 48
    cache = _gen((n_kv, max_seq, hd), 5, dev, torch.float16)
    ref = to_np(cache).copy()
    cur = 40
    for t in range(30):
        src = _gen((n_kv, 1, hd), 100 + t, dev)
        print(f"case kv_cache_update decode step {t} cur {cur}", flush=True)
        n = ops.kv_cache_update(src, cache, cur)
        assert n == orc.kv_cache_update(to_np(src), ref, 1, n_kv, 1, hd, max_seq, cur)
        _same(cache, ref, f"step {t}")
        cur = n


def test_kv_cache_update_rejects_bad_arguments(dev):
    from sapient_amd._lib import EINVAL, ERANGE, lib
    import ctypes
    cache = torch.arange(2 * 8 * 16, device=dev, dtype=torch.float32).reshape(2, 8, 16)
    before = cache.clone()
    src = torch.ones(2, 9, 16, device=dev)
    n = ctypes.c_int64(-7)
    s = torch.cuda.current_stream().cuda_stream
    L = lib()
    assert L.sph_kv_cache_update(src.data_ptr(), 0, cache.data_ptr(), 0, 2, 9, 16, 8, 0, ctypes.addressof(n), s) == ERANGE
    assert L.sph_kv_cache_update(src.data_ptr(), 0, cache.data_ptr(), 0, 2, 1, 16, 8, 9, ctypes.addressof(n), s) == EINVAL
    assert L.sph_kv_cache_update(src.data_ptr(), 0, cache.data_ptr(), 0, 2, 1, 16, 8, 2, None, s) == EINVAL
    assert L.sph_kv_cache_update(src.data_ptr(), 0, cache.data_ptr(), 0, 2, 1, 16, 8, -1, ctypes.addressof(n), s) == EINVAL
    # A full cache whose append would be rejected: the window must not slide either.
    assert L.sph_kv_cache_update(None, 0, cache.data_ptr(), 0, 2, 1, 16, 8, 8, ctypes.addressof(n), s) == EINVAL
    q8 = (torch.arange(2 * 8 * 34, device=dev) % 251).to(torch.uint8).reshape(2, 8, 34)
    q8_before = q8.clone()
    raw = torch.ones(2 * 32 + 4, device=dev)
    assert L.sph_kv_cache_update(raw.data_ptr() + 4, 0, q8.data_ptr(), 8, 2, 1, 32, 8, 8, ctypes.addressof(n), s) == EINVAL
    torch.cuda.synchronize()
    assert n.value == -7 and torch.equal(cache, before) and torch.equal(q8, q8_before)


# The out-of-place form (sph_kv_cache_update_into): the updated cache lands in a second buffer, which the
# caller then uses as its cache; the reference takes the cache as &mut Tensor (common.rs:355-359).
def _sentinel(shape, dtype, dev):
    """A buffer of a recognisable pattern, so rows the call must not touch can be checked."""
    n = 1
    for d in shape:
        n *= d
    if dtype == torch.uint8:
        return (torch.arange(n, device=dev) % 253).to(torch.uint8).reshape(shape)
    return (torch.arange(n, device=dev, dtype=torch.float32) * 0.5 - 7).to(dtype).reshape(shape)


def _check_into(cache, out, before_cache, before_out, want, n, what):
    """out rows [0, n) equal the oracle's cache rows [0, n) bit for bit, out rows past n are untouched, and
    the source cache is unchanged."""
    got = to_np(out)
    if got.dtype == np.float32:
        assert_bits_equal(got[:, :n], want[:, :n], what)
    else:
        assert np.array_equal(got[:, :n].view(np.uint8), want[:, :n].view(np.uint8)), what
    assert np.array_equal(got[:, n:].view(np.uint8), before_out[:, n:].view(np.uint8)), f"{what}: rows past {n}"
    assert np.array_equal(to_np(cache).view(np.uint8), before_cache.view(np.uint8)), f"{what}: source cache"


@pytest.mark.parametrize("cdtype", [torch.float32, torch.float16, torch.bfloat16], ids=IDS)
@pytest.mark.parametrize("n_kv,hd,max_seq,cur_len,seq", _UPD_CASES)
def test_kv_cache_update_into_matches_oracle(dev, orc, cdtype, n_kv, hd, max_seq, cur_len, seq):
    """The out-of-place update: rows [0, new_len) of out equal the in-place update's (the oracle's
    update_kv_cache) bit for bit, whatever the shift; rows past new_len and the source cache keep their bytes."""
    print(f"case kv_cache_update_into {cdtype} {n_kv}x{hd} max {max_seq} cur {cur_len} seq {seq}", flush=True)
    src = _gen((n_kv, seq, hd), seq * 7 + hd, dev)
    cache = _gen((n_kv, max_seq, hd), 17 + hd, dev, cdtype)
    out = _sentinel((n_kv, max_seq, hd), cdtype, dev)
    before_cache, before_out = to_np(cache).copy(), to_np(out).copy()
    want = before_cache.copy()
    n = ops.kv_cache_update_into(src, cache, out, cur_len)
    want_n = orc.kv_cache_update(to_np(src), want, CODE[cdtype], n_kv, seq, hd, max_seq, cur_len)
    assert n == want_n == min(cur_len + seq, max_seq)
    _check_into(cache, out, before_cache, before_out, want, n, f"kv_cache_update_into {cdtype}")


@pytest.mark.parametrize("sdtype,cdtype", [(torch.float16, torch.float32), (torch.bfloat16, torch.float32),
                                           (torch.float16, torch.float16), (torch.bfloat16, torch.float16),
                                           (torch.float32, torch.bfloat16), (torch.float16, torch.bfloat16)],
                         ids=lambda d: IDS(d))
@pytest.mark.parametrize("n_kv,hd,max_seq,cur_len,seq", [(8, 128, 1024, 1024, 1), (3, 64, 16, 12, 7),
                                                         (2, 64, 16, 5, 3), (5, 3, 40, 40, 2)])
def test_kv_cache_update_into_source_types(dev, orc, sdtype, cdtype, n_kv, hd, max_seq, cur_len, seq):
    """Every source type into every cache type (the fused launch widens or narrows the new rows)."""
    print(f"case kv_cache_update_into {sdtype}->{cdtype} {n_kv}x{hd} max {max_seq} cur {cur_len} seq {seq}",
          flush=True)
    src = _gen((n_kv, seq, hd), 3 * seq + hd, dev, sdtype)
    cache = _gen((n_kv, max_seq, hd), 29 + hd, dev, cdtype)
    out = _sentinel((n_kv, max_seq, hd), cdtype, dev)
    before_cache, before_out = to_np(cache).copy(), to_np(out).copy()
    want = before_cache.copy()
    n = ops.kv_cache_update_into(src, cache, out, cur_len)
    assert n == orc.kv_cache_update(widen(src, orc), want, CODE[cdtype], n_kv, seq, hd, max_seq, cur_len)
    _check_into(cache, out, before_cache, before_out, want, n, f"{sdtype}->{cdtype}")


@pytest.mark.parametrize("n_kv,hd,max_seq,cur_len,seq", [(2, 64, 16, 16, 1), (3, 32, 24, 20, 9), (8, 128, 512, 512, 1),
                                                         (2, 128, 64, 40, 64), (2, 64, 16, 3, 4)])
def test_kv_cache_update_into_q8_0(dev, orc, n_kv, hd, max_seq, cur_len, seq):
    """The quantized cache: kept 34-byte blocks moved as raw bytes into out, new rows quantized there."""
    print(f"case kv_cache_update_into q8_0 {n_kv}x{hd} max {max_seq} cur {cur_len} seq {seq}", flush=True)
    g = torch.Generator(device=dev).manual_seed(max_seq + cur_len)
    src = torch.randn(n_kv, seq, hd, generator=g, device=dev) * 3
    row = hd // 32 * 34
    cache = torch.randint(0, 256, (n_kv, max_seq, row), generator=g, device=dev, dtype=torch.int32).to(torch.uint8)
    out = _sentinel((n_kv, max_seq, row), torch.uint8, dev)
    before_cache, before_out = to_np(cache).copy(), to_np(out).copy()
    want = before_cache.copy()
    n = ops.kv_cache_update_into(src, cache, out, cur_len)
    assert n == orc.kv_cache_update(to_np(src), want, orc.Q8_0, n_kv, seq, hd, max_seq, cur_len)
    _check_into(cache, out, before_cache, before_out, want, n, "q8_0")


@pytest.mark.parametrize("cdtype", [torch.float16, torch.uint8], ids=IDS)
def test_kv_cache_update_into_decode_sequence(dev, orc, cdtype):
    """Thirty decode steps past a full cache, alternating between two buffers as a caller that installs
    each step's `out` as its cache would; every step checked against the oracle's in-place cache."""
    n_kv, hd, max_seq = 4, 64, 48
    q8 = cdtype == torch.uint8
    row = hd // 32 * 34 if q8 else hd
    if q8:
        g = torch.Generator(device=dev).manual_seed(5)
        cur_buf = torch.randint(0, 256, (n_kv, max_seq, row), generator=g, device=dev, dtype=torch.int32)
        cur_buf = cur_buf.to(torch.uint8)
    else:
        cur_buf = _gen((n_kv, max_seq, hd), 5, dev, cdtype)
    spare = _sentinel((n_kv, max_seq, row), cdtype, dev)
    ref = to_np(cur_buf).copy()
    cur = 40
    for t in range(30):
        src = _gen((n_kv, 1, hd), 100 + t, dev)
        print(f"case kv_cache_update_into {cdtype} decode step {t} cur {cur}", flush=True)
        n = ops.kv_cache_update_into(src, cur_buf, spare, cur)
        assert n == orc.kv_cache_update(to_np(src), ref, orc.Q8_0 if q8 else 1, n_kv, 1, hd, max_seq, cur)
        got = to_np(spare)
        assert np.array_equal(got[:, :n].view(np.uint8), ref[:, :n].view(np.uint8)), f"step {t}"
        cur_buf, spare = spare, cur_buf
        cur = n


@pytest.mark.parametrize("offset", [2, 4, 8])
def test_kv_cache_update_into_unaligned_buffers(dev, orc, offset):
    """Buffers off 16-byte alignment take the two-launch path (raw units as wide as the alignment allows)."""
    n_kv, hd, max_seq, cur_len, seq = 3, 64, 20, 20, 2
    print(f"case kv_cache_update_into f16 unaligned by {offset}", flush=True)
    el = n_kv * max_seq * hd
    cache_raw = _gen((el + 8,), 41, dev, torch.float16)
    out_raw = _sentinel((el + 8,), torch.float16, dev)
    cache = cache_raw[offset // 2:offset // 2 + el].view(n_kv, max_seq, hd)
    out = out_raw[offset // 2:offset // 2 + el].view(n_kv, max_seq, hd)
    src = _gen((n_kv, seq, hd), 43, dev)
    before_cache, before_out = to_np(cache).copy(), to_np(out).copy()
    want = before_cache.copy()
    n = ops.kv_cache_update_into(src, cache, out, cur_len)
    assert n == orc.kv_cache_update(to_np(src), want, 1, n_kv, seq, hd, max_seq, cur_len)
    _check_into(cache, out, before_cache, before_out, want, n, f"offset {offset}")
    assert torch.equal(out_raw[:offset // 2], _sentinel((el + 8,), torch.float16, dev)[:offset // 2])


def test_kv_cache_update_into_rejects_bad_arguments(dev):
    from sapient_amd._lib import EINVAL, ERANGE, lib
    import ctypes
    cache = torch.arange(2 * 8 * 16, device=dev, dtype=torch.float32).reshape(2, 8, 16)
    out = torch.full((2, 8, 16), 3.0, device=dev)
    before, out_before = cache.clone(), out.clone()
    src = torch.ones(2, 9, 16, device=dev)
    n = ctypes.c_int64(-7)
    s = torch.cuda.current_stream().cuda_stream
    L = lib()
    a = ctypes.addressof(n)
    c, o, x = cache.data_ptr(), out.data_ptr(), src.data_ptr()
    assert L.sph_kv_cache_update_into(x, 0, c, o, 0, 2, 9, 16, 8, 0, a, s) == ERANGE     # seq > max_seq
    assert L.sph_kv_cache_update_into(x, 0, c, o, 0, 2, 1, 16, 8, 9, a, s) == EINVAL     # cur_len > max_seq
    assert L.sph_kv_cache_update_into(x, 0, c, o, 0, 2, 1, 16, 8, 2, None, s) == EINVAL  # no new_len
    assert L.sph_kv_cache_update_into(x, 0, c, None, 0, 2, 1, 16, 8, 8, a, s) == EINVAL  # no out
    assert L.sph_kv_cache_update_into(x, 0, None, o, 0, 2, 1, 16, 8, 8, a, s) == EINVAL  # kept rows, no cache
    assert L.sph_kv_cache_update_into(None, 0, c, o, 0, 2, 1, 16, 8, 8, a, s) == EINVAL  # no src
    assert L.sph_kv_cache_update_into(x, 0, c, c, 0, 2, 1, 16, 8, 8, a, s) == EINVAL     # out is cache
    assert L.sph_kv_cache_update_into(x, 0, c, c + 64, 0, 2, 1, 16, 8, 8, a, s) == EINVAL  # out overlaps cache
    assert L.sph_kv_cache_update_into(o, 0, c, o, 0, 2, 1, 16, 8, 8, a, s) == EINVAL     # src inside out
    assert L.sph_kv_cache_update_into(x, 0, c, o, 8, 2, 1, 16, 8, 8, a, s) == EINVAL     # Q8_0 at hd 16
    torch.cuda.synchronize()
    assert n.value == -7 and torch.equal(cache, before) and torch.equal(out, out_before)
