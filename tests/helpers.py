"""Comparison helpers for parity tests: relative error, ulp distance of half
formats, and conversions between torch device tensors and numpy."""
from __future__ import annotations

import numpy as np
import torch


def to_np(t: torch.Tensor) -> np.ndarray:
    """Device or host tensor → numpy (f16/bf16 come back as uint16 bit patterns)."""
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.float16:
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def widen(t: torch.Tensor, orc) -> np.ndarray:
    """Exact f32 values of a tensor of any float dtype (via the oracle's half widening)."""
    a = to_np(t)
    if t.dtype == torch.float16:
        return orc.f16_bits_to_f32(a)
    if t.dtype == torch.bfloat16:
        return orc.bf16_bits_to_f32(a)
    return a.astype(np.float32, copy=False)


def narrow_bits(x: np.ndarray, dtype: torch.dtype, orc) -> np.ndarray:
    """Round f32 oracle results to the half format's bits (nearest-even)."""
    if dtype == torch.float16:
        return orc.f32_to_f16_bits(x)
    if dtype == torch.bfloat16:
        return orc.f32_to_bf16_bits(x)
    raise ValueError(dtype)


def _ordered16(bits: np.ndarray) -> np.ndarray:
    b = bits.astype(np.int32)
    return np.where(b & 0x8000, -(b & 0x7FFF), b & 0x7FFF)


def ulp_diff16(a_bits: np.ndarray, b_bits: np.ndarray, dtype: torch.dtype) -> np.ndarray:
    """Distance in representable values between two f16/bf16 bit arrays (NaN vs NaN = 0)."""
    a_bits, b_bits = np.asarray(a_bits, np.uint16), np.asarray(b_bits, np.uint16)
    if dtype == torch.float16:
        nan = lambda b: ((b & 0x7C00) == 0x7C00) & ((b & 0x3FF) != 0)
    else:
        nan = lambda b: ((b & 0x7F80) == 0x7F80) & ((b & 0x7F) != 0)
    d = np.abs(_ordered16(a_bits) - _ordered16(b_bits))
    both = nan(a_bits) & nan(b_bits)
    one = nan(a_bits) ^ nan(b_bits)
    d = np.where(both, 0, d)
    return np.where(one, 1 << 20, d)


def max_rel(got: np.ndarray, want: np.ndarray, floor: float = 0.0) -> float:
    """max |got - want| / max(|want|, floor); exact equality (incl. NaN==NaN) counts 0."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    same = (got == want) | (np.isnan(got) & np.isnan(want))
    den = np.maximum(np.abs(want), floor)
    with np.errstate(divide="ignore", invalid="ignore"):
        r = np.where(same, 0.0, np.abs(got - want) / den)
    r = np.where(np.isnan(r), np.inf, r)
    return float(r.max()) if r.size else 0.0


def assert_bits_equal(got: np.ndarray, want: np.ndarray, what: str) -> None:
    """Bit-exact f32 comparison; NaNs must match as NaNs (payload not compared)."""
    g = np.asarray(got, np.float32).reshape(-1)
    w = np.asarray(want, np.float32).reshape(-1)
    assert g.shape == w.shape, f"{what}: shape {g.shape} vs {w.shape}"
    gb, wb = g.view(np.uint32), w.view(np.uint32)
    nan_ok = np.isnan(g) & np.isnan(w)
    bad = (gb != wb) & ~nan_ok
    if bad.any():
        i = int(np.flatnonzero(bad)[0])
        raise AssertionError(f"{what}: {int(bad.sum())} of {g.size} differ; first at {i}: "
                             f"got {g[i]!r} ({gb[i]:#010x}) want {w[i]!r} ({wb[i]:#010x})")


def assert_bits16_equal(got: np.ndarray, want: np.ndarray, what: str) -> None:
    """Bit-exact comparison of f16/bf16 bit arrays, reporting the first mismatches."""
    g = np.asarray(got, np.uint16).reshape(-1)
    w = np.asarray(want, np.uint16).reshape(-1)
    assert g.shape == w.shape, f"{what}: shape {g.shape} vs {w.shape}"
    bad = np.flatnonzero(g != w)
    if bad.size:
        ex = ", ".join(f"[{i}] got {g[i]:#06x} want {w[i]:#06x}" for i in bad[:6])
        raise AssertionError(f"{what}: {bad.size} of {g.size} differ: {ex}")


def assert_ulp16(got: np.ndarray, want: np.ndarray, dtype, max_ulp: int, what: str) -> None:
    """f16/bf16 bits within max_ulp representable values, reporting the worst elements."""
    g = np.asarray(got, np.uint16).reshape(-1)
    w = np.asarray(want, np.uint16).reshape(-1)
    d = ulp_diff16(g, w, dtype)
    bad = np.flatnonzero(d > max_ulp)
    if bad.size:
        worst = bad[np.argsort(-d[bad])][:6]
        ex = ", ".join(f"[{i}] got {g[i]:#06x} want {w[i]:#06x} ({int(d[i])} ulp)" for i in worst)
        raise AssertionError(f"{what}: {bad.size} of {g.size} beyond {max_ulp} ulp: {ex}")


def layer_norm_bound(x32: np.ndarray, w, b, ref: np.ndarray) -> np.ndarray:
    """Per-element bound on |kernel - oracle| for LayerNorm: the kernel sums Σx and Σ(x − mean)² in
    another order than the reference's serial folds, which moves the mean and the variance by about
    2^-24·√n·(|mean| + σ) (8× that as the margin); everything else rounds alike."""
    x64 = x32.astype(np.float64)
    n = x64.shape[-1]
    mu = x64.mean(axis=-1, keepdims=True)
    sd = np.maximum(x64.std(axis=-1, keepdims=True), 1e-30)
    normed = np.abs(x64 - mu) / sd
    wa = 1.0 if w is None else np.abs(w.astype(np.float64))
    rel = 8 * 2.0 ** -24 * np.sqrt(n) * (np.abs(mu) + sd) / sd
    return wa * (1 + normed) * rel + 2.0 ** -22 * np.abs(ref.astype(np.float64)) + 1e-30


def check_layer_norm(out: torch.Tensor, ref: np.ndarray, x32, w, b, orc, what: str):
    """LayerNorm parity: f32 outputs within layer_norm_bound of the oracle; half outputs within 1 ulp
    of its f32 result rounded to nearest-even, or within that bound plus half an ulp."""
    bound = layer_norm_bound(x32, w, b, ref)
    if out.dtype == torch.float32:
        got = to_np(out).astype(np.float64)
        bad = ~(np.abs(got - ref) <= bound)
        assert not bad.any(), f"{what}: {int(bad.sum())} beyond bound; worst {np.max(np.abs(got - ref) / bound):.2f}x"
    else:
        got16 = to_np(out)
        want16 = narrow_bits(ref, out.dtype, orc)
        d = ulp_diff16(got16, want16, out.dtype).reshape(ref.shape)
        g32 = widen(out, orc).astype(np.float64)
        mant = 10 if out.dtype == torch.float16 else 7
        e = np.floor(np.log2(np.maximum(np.abs(ref.astype(np.float64)), 2.0 ** -14)))
        half_ulp = 0.5 * 2.0 ** (e - mant)
        ok = (d <= 1) | (np.abs(g32 - ref) <= bound + half_ulp)
        assert ok.all(), f"{what}: {int((~ok).sum())} of {ok.size} beyond 1 ulp and the f32 bound"
