"""GPU parity: token-embedding gather with GGUF row dequantization — bit-exact.

Reference: crates/sapient-models/src/forward/common.rs:164-217 (embed_tokens /
gather_row_f32), crates/sapient-core/src/tensor.rs:362-398, :421-467, :504-527,
:534-576 (Q4_0 / Q8_0 / Q4_K / Q5_K / Q6_K dequant). Every dequantized value
must equal the oracle's bits (NaN table entries: NaN-ness only).
"""
import numpy as np
import pytest
import torch

from helpers import assert_bits_equal, to_np
from refvec import (WgpuLcg, f16_bits, gather_test_values, quantize_q8_0_blocks, random_q4_k_blocks,
                    random_q6_k_blocks)

import sapient_amd.ops as ops
from sapient_amd._lib import BF16, F16, F32, Q4_0, Q4_K, Q5_K, Q6_K, Q8_0

pytestmark = pytest.mark.gpu


def _dev_bytes(a: np.ndarray, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.uint8).reshape(-1).copy()).to(dev)


def _ids(ids, dev) -> torch.Tensor:
    return torch.from_numpy(np.asarray(ids, np.uint32).view(np.int32).copy()).to(dev)


def _gather(dev, table_bytes: np.ndarray, dt: int, vocab: int, hidden: int, ids) -> np.ndarray:
    out = ops.embed(_dev_bytes(table_bytes, dev), dt, vocab, hidden, _ids(ids, dev))
    return to_np(out)


def test_embed_q8_0_matches_wgpu_test_vectors(dev, orc):
    """resident.rs:565-592: vocab 100 x 320, lcg 0x9E3779B9, ids [7, 0, 99, 42]."""
    vocab, dim = 100, 320
    table = WgpuLcg().take(vocab * dim)
    blocks, deq = quantize_q8_0_blocks(table)
    ids = [7, 0, 99, 42]
    print("case embed q8_0 wgpu-vectors", flush=True)
    got = _gather(dev, blocks, Q8_0, vocab, dim, ids)
    want = deq.reshape(vocab, dim)[ids]
    assert_bits_equal(got, want, "embed_q8_0 vs test restatement")
    assert_bits_equal(got, orc.embed_tokens(blocks, Q8_0, vocab, dim, ids), "embed_q8_0 vs oracle")


def test_embed_q4_k_matches_wgpu_test_vectors(dev, orc):
    """resident.rs:678-705: vocab 50 x 512, random_q4_k_blocks, ids [3, 0, 49, 21]."""
    vocab, dim = 50, 512
    blocks, deq = random_q4_k_blocks(vocab * dim // 256, WgpuLcg())
    ids = [3, 0, 49, 21]
    print("case embed q4_k wgpu-vectors", flush=True)
    got = _gather(dev, blocks, Q4_K, vocab, dim, ids)
    assert_bits_equal(got, deq.reshape(vocab, dim)[ids], "embed_q4_k vs test restatement")


def test_embed_q6_k_matches_wgpu_test_vectors(dev, orc):
    """resident.rs:712-804 data generator (random_q6_k_blocks), vocab 40 x 512."""
    vocab, dim = 40, 512
    blocks, deq = random_q6_k_blocks(vocab * dim // 256, WgpuLcg())
    ids = [39, 0, 17, 5, 17]
    print("case embed q6_k wgpu-vectors", flush=True)
    got = _gather(dev, blocks, Q6_K, vocab, dim, ids)
    assert_bits_equal(got, deq.reshape(vocab, dim)[ids], "embed_q6_k vs test restatement")


def test_embed_row_gather_matches_full_dequant(dev, orc):
    """common.rs:678-718: vocab 17 x 256, LCG seed 0xABCD, ids [0, 7, 16, 3], F32 / F16 / Q8_0 tables."""
    vocab, hidden = 17, 256
    data = gather_test_values(vocab, hidden)
    ids = [0, 7, 16, 3]
    q8 = orc.quantize_q8_0(data)
    for dt, table, full in ((F32, data, data.reshape(-1)),
                            (F16, f16_bits(data), orc.f16_bits_to_f32(f16_bits(data))),
                            (Q8_0, q8, orc.dequant(q8, Q8_0, vocab * hidden))):
        print(f"case embed gather-vs-full dtype {dt}", flush=True)
        got = _gather(dev, table, dt, vocab, hidden, ids)
        assert_bits_equal(got, full.reshape(vocab, hidden)[ids], f"dtype {dt}")


@pytest.mark.parametrize("dt", [F16, BF16])
def test_embed_half_tables_all_bit_patterns(dev, orc, dt):
    """Every 16-bit pattern once: widening is exact (NaN payload aside)."""
    vocab, hidden = 256, 256
    table = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ids = list(range(vocab))[::-1]
    print(f"case embed all-bit-patterns {dt}", flush=True)
    got = _gather(dev, table, dt, vocab, hidden, ids)
    assert_bits_equal(got, orc.embed_tokens(table, dt, vocab, hidden, ids), f"widen {dt}")


def test_embed_q4_k_both_scale_branches_and_subnormal_scales(dev, orc):
    """Hand-built blocks: every 6-bit (sc, m) on both get_scale_min_k4 branches
    (j < 4 and j >= 4 with the high bits), with subnormal, tiny and large f16 d/dmin."""
    rng = np.random.default_rng(5)
    nb = 64
    blocks = rng.integers(0, 256, (nb, 144), dtype=np.uint8)
    dvals = np.array([0x0001, 0x03FF, 0x0400, 0x3C00, 0x7BFF, 0x1234], np.uint16)
    for b in range(nb):
        blocks[b, 0:2] = np.array([dvals[b % 6]], np.uint16).view(np.uint8)
        blocks[b, 2:4] = np.array([dvals[(b + 3) % 6]], np.uint16).view(np.uint8)
        blocks[b, 4:16] = (np.arange(12) * 21 + b * 7) % 256
    vocab, dim = nb // 4, 1024
    ids = list(range(vocab))
    got = _gather(dev, blocks, Q4_K, vocab, dim, ids)
    assert_bits_equal(got, orc.embed_tokens(blocks, Q4_K, vocab, dim, ids), "q4_k hand-built")


def _k_quant_headers(blocks: np.ndarray, dvals: np.ndarray) -> None:
    """d and dmin cycling through subnormal, tiny, one, large and negative f16 values; scale bytes that
    hit both get_scale_min_k4 branches with every high-bit combination."""
    nb = blocks.shape[0]
    for b in range(nb):
        blocks[b, 0:2] = np.array([dvals[b % len(dvals)]], np.uint16).view(np.uint8)
        blocks[b, 2:4] = np.array([dvals[(b + 3) % len(dvals)]], np.uint16).view(np.uint8)
        blocks[b, 4:16] = (np.arange(12) * 21 + b * 7) % 256


def test_embed_q5_k_bit_planes_scale_branches_and_reference_kat(dev, orc):
    """Q5_K (tensor.rs:421-467): random nibbles and high-bit planes under hand-built headers; the reference's
    KAT block (tensor.rs:800-830); and one qh bit at a time, which must move exactly one element."""
    rng = np.random.default_rng(6)
    nb = 64
    blocks = rng.integers(0, 256, (nb, 176), dtype=np.uint8)
    _k_quant_headers(blocks, np.array([0x0001, 0x03FF, 0x0400, 0x3C00, 0x7BFF, 0x1234, 0x8400], np.uint16))
    vocab, dim = nb // 4, 1024
    ids = list(range(vocab))[::-1]
    print("case embed q5_k hand-built", flush=True)
    got = _gather(dev, blocks, Q5_K, vocab, dim, ids)
    assert_bits_equal(got, orc.embed_tokens(blocks, Q5_K, vocab, dim, ids), "q5_k hand-built")
    # 256 one-bit blocks: block 8l + p sets bit p of qh[l] (d = 1, sc = 1, m = 0)
    planes = np.zeros((256, 176), np.uint8)
    planes[:, 0:2] = np.array([np.float16(1.0)]).view(np.uint8)
    planes[:, 4:8], planes[:, 12:16] = 1, 1
    for l in range(32):
        for p in range(8):
            planes[8 * l + p, 16 + l] = 1 << p
    got = _gather(dev, planes, Q5_K, 256, 256, list(range(256)))
    want = np.zeros((256, 256), np.float32)
    for l in range(32):
        for p in range(8):
            want[8 * l + p, 64 * (p // 2) + 32 * (p % 2) + l] = 16.0
    assert_bits_equal(got, want, "q5_k bit planes")
    kat = np.zeros(176, np.uint8)
    kat[0:2] = np.array([np.float16(1.0)]).view(np.uint8)
    kat[4:8], kat[12:16], kat[16 + 5], kat[16 + 0], kat[48 + 3] = 1, 1, 0b1, 0b100, 0x02
    y = _gather(dev, kat, Q5_K, 1, 256, [0]).reshape(-1)
    assert y[3] == 2.0 and y[5] == 16.0 and y[64] == 16.0 and np.count_nonzero(y) == 3


def test_embed_q4_0_every_byte_at_every_position(dev, orc):
    """Q4_0 (tensor.rs:362-376, the ggml split nibble order): all 256 byte values at each of the 16 byte
    positions under six scales (subnormal, one, negative, largest)."""
    blocks = []
    for dv in np.array([0x0001, 0x03FF, 0x3C00, 0xBC00, 0x7BFF, 0x2E66], np.uint16):
        for j in range(16):
            b = np.zeros((256, 18), np.uint8)
            b[:, 0:2] = np.array([dv], np.uint16).view(np.uint8)
            b[:, 2:] = np.random.default_rng(int(dv) + j).integers(0, 256, (256, 16), dtype=np.uint8)
            b[:, 2 + j] = np.arange(256, dtype=np.uint32).astype(np.uint8)
            blocks.append(b)
    blocks = np.concatenate(blocks)                       # 24576 blocks: vocab 3072 x hidden 256
    vocab, hidden = blocks.shape[0] * 32 // 256, 256
    ids = np.random.default_rng(7).permutation(vocab)
    print("case embed q4_0 every byte", flush=True)
    got = _gather(dev, blocks, Q4_0, vocab, hidden, ids)
    assert_bits_equal(got, orc.embed_tokens(blocks, Q4_0, vocab, hidden, ids), "q4_0")


@pytest.mark.parametrize("dt,block,nbytes", [(Q4_0, 32, 18), (Q5_K, 256, 176)], ids=["q4_0", "q5_k"])
def test_embed_new_formats_model_shape(dev, orc, dt, block, nbytes):
    """A Llama-3.2-1B-shaped table (vocab 128256 x 2048) with 8192 uniform ids — the whole gather bit-exact."""
    vocab, hidden, n = 128256, 2048, 8192
    rng = np.random.default_rng(8)
    nb = vocab * hidden // block
    table = rng.integers(0, 256, (nb, nbytes), dtype=np.uint8)
    hdr = 4 if dt == Q5_K else 2
    table[:, 0:hdr] = np.frombuffer(rng.uniform(0.0005, 0.02, nb * hdr // 2).astype(np.float16).tobytes(),
                                    np.uint8).reshape(nb, hdr)
    ids = rng.integers(0, vocab, n).astype(np.uint32)
    print(f"case embed {dt} {vocab}x{hidden} {n} ids", flush=True)
    got = _gather(dev, table, dt, vocab, hidden, ids)
    assert_bits_equal(got, orc.embed_tokens(table, dt, vocab, hidden, ids), f"{dt} model shape")


def test_embed_q8_0_every_quant_value(dev, orc):
    """All 256 int8 quants under f16 scales incl. subnormal / max / negative."""
    scales = np.array([0x0001, 0x0200, 0x3C00, 0xBC00, 0x7BFF, 0x2E66, 0x1000, 0x8001], np.uint16)
    blocks = np.zeros((8, 8, 34), np.uint8)  # 8 rows of 8 blocks: each row sweeps all 256 quants
    for r in range(8):
        for b in range(8):
            blocks[r, b, 0:2] = np.array([scales[(r + b) % 8]], np.uint16).view(np.uint8)
            blocks[r, b, 2:] = np.arange(32 * b, 32 * b + 32) % 256
    ids = [7, 3, 0, 5]
    got = _gather(dev, blocks, Q8_0, 8, 256, ids)
    assert_bits_equal(got, orc.embed_tokens(blocks, Q8_0, 8, 256, ids), "q8_0 sweep")


def _q4k_table(vocab, hidden, seed, dev):
    """Synthetic Q4_K table on the device: d, dmin ~U(0.0005, 0.02) as f16, scales and
    nibbles uniform random bytes."""
    g = torch.Generator(device=dev).manual_seed(seed)
    nb = vocab * hidden // 256
    t = torch.randint(0, 256, (nb, 144), generator=g, device=dev, dtype=torch.int32).to(torch.uint8)
    d = (torch.rand((nb, 2), generator=g, device=dev) * (0.02 - 0.0005) + 0.0005).to(torch.float16)
    t[:, 0:4] = d.view(torch.uint8).view(nb, 4)
    return t.reshape(-1)


def test_embed_q8_0_qwen_shape(dev, orc):
    """Qwen2.5-0.5B table 151936 x 896 Q8_0, T = 512 uniform ids (and T = 1)."""
    vocab, hidden = 151936, 896
    g = torch.Generator(device=dev).manual_seed(71)
    nb = vocab * hidden // 32
    t = torch.randint(-127, 128, (nb, 34), generator=g, device=dev, dtype=torch.int32).to(torch.int8).view(torch.uint8)
    d = (torch.rand((nb, 1), generator=g, device=dev) * (0.05 - 0.001) + 0.001).to(torch.float16)
    t[:, 0:2] = d.view(torch.uint8).view(nb, 2)
    table = t.reshape(-1).contiguous()
    tab_np = to_np(table)
    for T in (1, 512):
        ids = np.random.default_rng(T).integers(0, vocab, T).astype(np.uint32)
        print(f"case embed q8_0 qwen T={T}", flush=True)
        got = to_np(ops.embed(table, Q8_0, vocab, hidden, _ids(ids, dev)))
        assert_bits_equal(got, orc.embed_tokens(tab_np, Q8_0, vocab, hidden, ids), f"q8_0 T={T}")


@pytest.mark.parametrize("dist", ["uniform", "zipf"])
def test_embed_q4_k_llama3_full(dev, orc, dist):
    """128256 x 4096 Q4_K table, 65536 ids (uniform and Zipf s = 1.1): every row bit-exact."""
    vocab, hidden, n = 128256, 4096, 65536
    table = _q4k_table(vocab, hidden, 81, dev)
    rng = np.random.default_rng(82)
    if dist == "uniform":
        ids = rng.integers(0, vocab, n).astype(np.uint32)
    else:
        p = 1.0 / np.arange(1, vocab + 1) ** 1.1
        ranks = np.searchsorted(np.cumsum(p / p.sum()), rng.random(n))
        ids = rng.permutation(vocab)[np.minimum(ranks, vocab - 1)].astype(np.uint32)
    print(f"case embed q4_k full {dist}", flush=True)
    out = ops.embed(table, Q4_K, vocab, hidden, _ids(ids, dev))
    torch.cuda.synchronize()
    assert_bits_equal(to_np(out), orc.embed_tokens(to_np(table), Q4_K, vocab, hidden, ids), f"q4_k {dist}")


def test_embed_out_of_range_id_sets_flag_and_zero_fills(dev, orc):
    """common.rs:171-173 rejects ids >= vocab; the device path never reads the table for them."""
    vocab, hidden = 17, 256
    data = gather_test_values(vocab, hidden)
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    out = ops.embed(_dev_bytes(data, dev), F32, vocab, hidden, _ids([3, 17, 0xFFFFFFFF, 5], dev), bad_id_flag=flag)
    o = to_np(out)
    assert flag.item() == 1
    assert (o[1] == 0).all() and (o[2] == 0).all()
    assert_bits_equal(o[[0, 3]], data[[3, 5]], "valid rows")
    from oracle import ERANGE, OracleError
    with pytest.raises(OracleError) as e:
        orc.embed_tokens(data, F32, vocab, hidden, [17])
    assert e.value.status == ERANGE


def test_embed_rejects_bad_arguments(dev):
    from sapient_amd._lib import EINVAL, lib
    L = lib()
    t = torch.zeros(1024, dtype=torch.uint8, device=dev)
    ids = torch.zeros(2, dtype=torch.int32, device=dev)
    out = torch.zeros(2, 512, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    assert L.sph_embed(t.data_ptr(), Q8_0, 1, 48, ids.data_ptr(), 2, out.data_ptr(), None, s) == EINVAL  # 48 % 32
    assert L.sph_embed(t.data_ptr(), Q4_K, 1, 300, ids.data_ptr(), 2, out.data_ptr(), None, s) == EINVAL  # % 256
    assert L.sph_embed(t.data_ptr(), 3, 1, 256, ids.data_ptr(), 2, out.data_ptr(), None, s) == EINVAL    # Q4_1
    assert L.sph_embed(t.data_ptr(), Q4_0, 1, 48, ids.data_ptr(), 2, out.data_ptr(), None, s) == EINVAL  # 48 % 32
    assert L.sph_embed(t.data_ptr() + 2, Q5_K, 1, 256, ids.data_ptr(), 2, out.data_ptr(), None, s) == EINVAL
    assert L.sph_embed(t.data_ptr() + 1, Q4_K, 1, 256, ids.data_ptr(), 2, out.data_ptr(), None, s) == EINVAL


@pytest.mark.parametrize("hidden", [96, 320, 896, 4096, 8448])
@pytest.mark.parametrize("offset", [0, 2, 4, 8])
def test_embed_q8_0_every_staging_width(dev, orc, hidden, offset):
    """Q8_0 rows are staged through LDS with 16-, 8- or 4-byte loads, whichever divides both the row
    length and the table address, and read in place otherwise: widths 96 (102-byte rows: in place),
    320 (4-byte), 896 (8-byte), 4096 (16-byte), 8448 (16-byte, three chunks), each with the table
    shifted by 0, 2, 4 and 8 bytes, and one out-of-range id (zero row, flag raised)."""
    vocab = 64
    rng = np.random.default_rng(hidden + offset)
    nb = vocab * hidden // 32
    blocks = rng.integers(0, 256, (nb, 34), dtype=np.uint8)
    blocks[:, 0:2] = np.frombuffer(rng.uniform(-0.05, 0.05, nb).astype(np.float16).tobytes(), np.uint8).reshape(nb, 2)
    raw = torch.zeros(nb * 34 + 16, dtype=torch.uint8, device=dev)
    table = raw[offset:offset + nb * 34]
    table.copy_(torch.from_numpy(blocks.reshape(-1)).to(dev))
    ids = np.array(list(rng.permutation(vocab)[:40]) + [vocab + 5, 0, vocab - 1], np.uint32)
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    print(f"case embed q8_0 staging hidden {hidden} offset {offset}", flush=True)
    out = to_np(ops.embed(table, Q8_0, vocab, hidden, _ids(ids, dev), bad_id_flag=flag))
    ok = ids < vocab
    assert flag.item() == 1
    assert (out[~ok] == 0).all()
    assert_bits_equal(out[ok], orc.embed_tokens(blocks, Q8_0, vocab, hidden, ids[ok]), f"q8_0 {hidden} +{offset}")


_FORMATS = {  # dtype: (elements per block, bytes per block, f16 scale byte offsets, table alignment the ABI needs)
    "q4_0": (Q4_0, 32, 18, (0,), 2), "q5_k": (Q5_K, 256, 176, (0, 2), 16), "q6_k": (Q6_K, 256, 210, (208,), 2),
    "f16": (F16, 4, 8, (), 8), "bf16": (BF16, 4, 8, (), 8), "f32": (F32, 4, 16, (), 16),
}
_WIDTHS = {"q4_0": (32, 64, 128, 4096, 8448), "q5_k": (256, 4096, 8448), "q6_k": (256, 512, 1024, 2048, 8192),
           "f16": (4, 8, 3000), "bf16": (2600,), "f32": (4, 4100)}


@pytest.mark.parametrize("fmt,hidden,offset", [(f, h, o) for f, hs in _WIDTHS.items() for h in hs
                                               for o in (0, 2, 4, 8) if o % _FORMATS[f][4] == 0])
def test_embed_every_format_every_staging_width(dev, orc, fmt, hidden, offset):
    """Every table type but Q4_K is staged through LDS with 16-, 8- or 4-byte loads, whichever divides both
    the row length and the table address, and read in place otherwise; rows longer than one staging chunk
    (4608 bytes) take several. Widths chosen per format to reach each load width, a single block, one
    chunk and several chunks; the table shifted by each offset its alignment allows; one out-of-range id
    (zero row, flag raised). Bar: bit-exact with the oracle."""
    dt, blk, nbytes, scale_offs, _ = _FORMATS[fmt]
    vocab = 48
    rng = np.random.default_rng(hidden * 16 + offset)
    nb = vocab * hidden // blk
    blocks = rng.integers(0, 256, (nb, nbytes), dtype=np.uint8)
    for so in scale_offs:
        blocks[:, so:so + 2] = np.frombuffer(rng.uniform(-0.05, 0.05, nb).astype(np.float16).tobytes(),
                                             np.uint8).reshape(nb, 2)
    raw = torch.zeros(nb * nbytes + 16, dtype=torch.uint8, device=dev)
    table = raw[offset:offset + nb * nbytes]
    table.copy_(torch.from_numpy(blocks.reshape(-1)).to(dev))
    ids = np.array(list(rng.permutation(vocab)[:30]) + [vocab + 7, 0, vocab - 1, 3, 3], np.uint32)
    flag = torch.zeros(1, dtype=torch.int32, device=dev)
    print(f"case embed {fmt} staging hidden {hidden} offset {offset}", flush=True)
    out = to_np(ops.embed(table, dt, vocab, hidden, _ids(ids, dev), bad_id_flag=flag))
    ok = ids < vocab
    assert flag.item() == 1
    assert (out[~ok] == 0).all()
    assert_bits_equal(out[ok], orc.embed_tokens(blocks, dt, vocab, hidden, ids[ok]), f"{fmt} {hidden} +{offset}")
