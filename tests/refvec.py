"""Input generators and in-test expectations of the reference's own tests,
restated in numpy so their vectors can be rebuilt bit for bit.

Sources (paths relative to the sapient workspace root):
- crates/sapient-models/src/forward/common.rs:678-718
  (embed_row_gather_matches_full_dequant: LCG seed 0xABCD, (s >> 40) / 2^24 * 2 - 1)
- crates/sapient-backends/wgpu/tests/resident.rs:36-42, :61-69
  (LCG seeds 0x12345678 / 0x9E3779B9, (s >> 33) as f32 / u32::MAX as f32 * 2 - 1)
- resident.rs:506-524 (quantize_q8_0_blocks), :600-640 (random_q4_k_blocks),
  :712-738 (random_q6_k_blocks)
- crates/sapient-backends/cpu/src/kernels/quant.rs:223-235 (quantize_q8_0_block)
"""
from __future__ import annotations

import numpy as np

_MUL = 6364136223846793005
_INC = 1442695040888963407
_M64 = (1 << 64) - 1
_U32MAX_F32 = np.float32(4294967295.0)  # `u32::MAX as f32` rounds to 2^32


def lcg_states(seed: int, n: int) -> np.ndarray:
    """The first n updated states of s = s*MUL + INC (mod 2^64)."""
    out = np.empty(n, np.uint64)
    s = seed
    for i in range(n):
        s = (s * _MUL + _INC) & _M64
        out[i] = s
    return out


class WgpuLcg:
    """resident.rs `lcg()` / the rms_norm test's inline generator: a stream of f32 in [-1, 1]."""

    def __init__(self, seed: int = 0x9E3779B9):
        self.s = seed

    def take(self, n: int) -> np.ndarray:
        out = np.empty(n, np.float32)
        s = self.s
        for i in range(n):
            s = (s * _MUL + _INC) & _M64
            out[i] = np.float32(s >> 33)
        self.s = s
        return (out / _U32MAX_F32) * np.float32(2.0) - np.float32(1.0)

    def __call__(self) -> np.float32:
        return self.take(1)[0]


def gather_test_values(vocab: int = 17, hidden: int = 256, seed: int = 0xABCD) -> np.ndarray:
    """common.rs:681-688: ((s >> 40) as f32 / (1 << 24) as f32) * 2.0 - 1.0."""
    st = lcg_states(seed, vocab * hidden)
    v = (st >> np.uint64(40)).astype(np.float32) / np.float32(1 << 24)
    return (v * np.float32(2.0) - np.float32(1.0)).reshape(vocab, hidden)


def f16_bits(x: np.ndarray) -> np.ndarray:
    """half::f16::from_f32 (round to nearest even), via numpy's IEEE conversion."""
    return np.asarray(x, np.float32).astype(np.float16).view(np.uint16)


def _as_u8_trunc(v: np.ndarray) -> np.ndarray:
    """Rust `f as u8`: truncate toward zero, saturate to [0, 255]."""
    return np.clip(np.trunc(v), 0, 255).astype(np.uint8)


def _as_i8_trunc(v: np.ndarray) -> np.ndarray:
    """Rust `f as i8`: truncate toward zero, saturate to [-128, 127]."""
    return np.clip(np.trunc(v), -128, 127).astype(np.int8)


def quantize_q8_0_blocks(w: np.ndarray):
    """resident.rs:506-524 / quant.rs:223-235 → (block bytes, dequantized values)."""
    w = np.asarray(w, np.float32).reshape(-1, 32)
    amax = np.max(np.abs(w), axis=1)
    d = (amax / np.float32(127.0)).astype(np.float32)
    inv = np.where(d > 0, np.float32(1.0) / np.where(d > 0, d, np.float32(1.0)), np.float32(0.0)).astype(np.float32)
    d16 = f16_bits(d)
    scaled = (w * inv[:, None]).astype(np.float32)
    t = np.trunc(scaled)  # f32::round: half away from zero (scaled - t is exact)
    rounded = t + np.where(np.abs(scaled - t) >= np.float32(0.5), np.sign(scaled), np.float32(0.0))
    q = np.clip(rounded, -127, 127).astype(np.int8)
    blocks = np.empty((w.shape[0], 34), np.uint8)
    blocks[:, 0:2] = d16.reshape(-1, 1).view(np.uint8).reshape(-1, 2)
    blocks[:, 2:] = q.view(np.uint8)
    scale = d16.view(np.float16).astype(np.float32)
    deq = (scale[:, None] * q.astype(np.float32)).astype(np.float32)
    return blocks.reshape(-1), deq.reshape(-1)


def _scale_min_k4(j: int, s: np.ndarray):
    if j < 4:
        return s[j] & 63, s[j + 4] & 63
    return (s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4), (s[j + 4] >> 4) | ((s[j] >> 6) << 4)


def random_q4_k_blocks(nblocks: int, nxt: WgpuLcg):
    """resident.rs:600-640 → (block bytes, dequantized values by that test's own formula)."""
    blocks = np.empty((nblocks, 144), np.uint8)
    deq = np.empty((nblocks, 256), np.float32)
    for b in range(nblocks):
        d = f16_bits(np.float32(1.0e-4) * (np.float32(1.0) + abs(nxt())))
        dmin = f16_bits(np.float32(1.0e-4) * (np.float32(1.0) + abs(nxt())))
        blocks[b, 0:2] = np.array([d], np.uint16).view(np.uint8)
        blocks[b, 2:4] = np.array([dmin], np.uint16).view(np.uint8)
        blocks[b, 4:16] = _as_u8_trunc(np.abs(nxt.take(12)) * np.float32(255.0))
        blocks[b, 16:144] = _as_u8_trunc(np.abs(nxt.take(128)) * np.float32(255.0))
        scales, qs = blocks[b, 4:16].astype(np.int64), blocks[b, 16:144]
        df = np.float32(np.array([d], np.uint16).view(np.float16)[0])
        mf = np.float32(np.array([dmin], np.uint16).view(np.float16)[0])
        for is_ in range(8):
            sc, mn = _scale_min_k4(is_, scales)
            d1, m1 = np.float32(df * np.float32(sc)), np.float32(mf * np.float32(mn))
            byte = qs[(is_ // 2) * 32:(is_ // 2) * 32 + 32]
            q = (byte & 0xF) if is_ % 2 == 0 else (byte >> 4)
            deq[b, 32 * is_:32 * is_ + 32] = (d1 * q.astype(np.float32)).astype(np.float32) - m1
    return blocks.reshape(-1), deq.reshape(-1)


def random_q6_k_blocks(nblocks: int, nxt: WgpuLcg):
    """resident.rs:712-738 → (block bytes, dequantized values by that test's own formula)."""
    blocks = np.empty((nblocks, 210), np.uint8)
    deq = np.empty((nblocks, 256), np.float32)
    e = np.arange(256)
    h, r = e // 128, e % 128
    g, l = r // 32, r % 32
    for b in range(nblocks):
        blocks[b, 0:192] = _as_u8_trunc(np.abs(nxt.take(192)) * np.float32(255.0))
        blocks[b, 192:208] = _as_i8_trunc(nxt.take(16) * np.float32(127.0)).view(np.uint8)
        d = f16_bits(np.float32(2.0e-5) * (np.float32(1.0) + abs(nxt())))
        blocks[b, 208:210] = np.array([d], np.uint16).view(np.uint8)
        ql, qh, sc = blocks[b, 0:128], blocks[b, 128:192], blocks[b, 192:208].view(np.int8)
        df = np.float32(np.array([d], np.uint16).view(np.float16)[0])
        q = ((ql[h * 64 + (g % 2) * 32 + l] >> ((g // 2) * 4)) & 0xF) | (((qh[h * 32 + l] >> (g * 2)) & 3) << 4)
        scale = sc[h * 8 + 2 * g + l // 16].astype(np.float32)
        deq[b] = ((df * scale).astype(np.float32) * (q.astype(np.int32) - 32).astype(np.float32)).astype(np.float32)
    return blocks.reshape(-1), deq.reshape(-1)
