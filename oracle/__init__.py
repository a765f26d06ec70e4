"""numpy wrappers over the CPU oracle (``liboracle.so``, built from
``oracle/sapient_oracle.c`` by ``oracle/Makefile``).

Test infrastructure only: the test suite, the smoke check and the benchmark's
CPU-baseline leg use it as the reference for results. It is never part of the product path.
Every wrapper takes and returns numpy arrays; dtypes follow the reference's
CPU kernels (f32 compute, f32 outputs).
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

# GGUF tensor type ids (crates/sapient-io/src/gguf.rs:90-104)
F32, F16, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K, BF16 = 0, 1, 2, 8, 12, 13, 14, 30
OK, EINVAL, ERANGE = 0, -1, -3

_lib = None


def build() -> Path:
    """Compile liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = C.CDLL(str(LIB_PATH))
        vp, sz, fl = C.c_void_p, C.c_size_t, C.c_float
        sig = {
            "sor_f16_to_f32_n": (None, [vp, vp, sz]),
            "sor_f32_to_f16_n": (None, [vp, vp, sz]),
            "sor_bf16_to_f32_n": (None, [vp, vp, sz]),
            "sor_f32_to_bf16_n": (None, [vp, vp, sz]),
            "sor_rms_norm": (None, [vp, vp, vp, sz, sz, fl]),
            "sor_add": (C.c_int, [vp, sz, vp, sz, vp]),
            "sor_mul": (C.c_int, [vp, sz, vp, sz, vp]),
            "sor_add_rms_norm": (None, [vp, vp, vp, vp, vp, sz, sz, fl]),
            "sor_layer_norm": (None, [vp, vp, vp, vp, sz, sz, fl]),
            "sor_add_bias_last_dim": (None, [vp, vp, vp, sz, sz]),
            "sor_silu": (None, [vp, vp, sz]),
            "sor_swiglu": (None, [vp, vp, vp, sz]),
            "sor_gelu": (None, [vp, vp, sz]),
            "sor_gelu_erf": (None, [vp, vp, sz]),
            "sor_apply_rope": (C.c_int, [vp, vp, sz, sz, sz, sz, vp, sz, fl]),
            "sor_apply_rope_partial_scaled": (C.c_int, [vp, vp, sz, sz, sz, sz, vp, sz, fl, sz, fl]),
            "sor_apply_rope_interleaved": (C.c_int, [vp, vp, sz, sz, sz, sz, vp, sz, fl, sz, fl]),
            "sor_unpermute_qk_rows": (C.c_int, [vp, vp, sz, sz, sz]),
            "sor_dequant_q4_0": (None, [vp, sz, vp]),
            "sor_dequant_q8_0": (None, [vp, sz, vp]),
            "sor_dequant_q4_k": (None, [vp, sz, vp]),
            "sor_dequant_q5_k": (None, [vp, sz, vp]),
            "sor_dequant_q6_k": (None, [vp, sz, vp]),
            "sor_row_bytes": (sz, [C.c_int, sz]),
            "sor_embed_tokens": (C.c_int, [vp, C.c_int, sz, sz, vp, sz, vp]),
            "sor_quantize_q8_0": (None, [vp, sz, vp]),
            "sor_transpose_heads": (None, [vp, vp, sz, sz, sz, sz]),
            "sor_kv_append": (C.c_int, [vp, vp, C.c_int, sz, sz, sz, sz, sz]),
            "sor_kv_cache_update": (C.c_int, [vp, vp, C.c_int, sz, sz, sz, sz, sz, C.POINTER(sz)]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


class OracleError(RuntimeError):
    def __init__(self, status: int, what: str):
        super().__init__(f"{what}: oracle status {status}")
        self.status = status


# ── half conversions ─────────────────────────────────────────────────────────
def f16_bits_to_f32(bits) -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(b.shape, np.float32)
    lib().sor_f16_to_f32_n(_p(b), _p(out), b.size)
    return out


def f32_to_f16_bits(x) -> np.ndarray:
    x = _f32(x)
    out = np.empty(x.shape, np.uint16)
    lib().sor_f32_to_f16_n(_p(x), _p(out), x.size)
    return out


def bf16_bits_to_f32(bits) -> np.ndarray:
    b = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(b.shape, np.float32)
    lib().sor_bf16_to_f32_n(_p(b), _p(out), b.size)
    return out


def f32_to_bf16_bits(x) -> np.ndarray:
    x = _f32(x)
    out = np.empty(x.shape, np.uint16)
    lib().sor_f32_to_bf16_n(_p(x), _p(out), x.size)
    return out


# ── ops ──────────────────────────────────────────────────────────────────────
def rms_norm(x, weight, eps: float) -> np.ndarray:
    x = _f32(x)
    w = None if weight is None else _f32(weight)
    dim = x.shape[-1] if x.ndim else 1
    outer = x.size // dim if dim else 0
    out = np.empty_like(x)
    lib().sor_rms_norm(_p(x), None if w is None else _p(w), _p(out), outer, dim, np.float32(eps))
    return out


def add_rms_norm(x, residual, weight, eps: float):
    """(normed, updated residual) of add (llama.rs:508) then rms_norm (llama.rs:515); weight may be
    None (unit weight, as rms_norm's)."""
    x, r = _f32(x), _f32(residual)
    w = None if weight is None else _f32(weight)
    dim = x.shape[-1]
    if r.shape != x.shape or (w is not None and w.size != dim):
        raise ValueError("residual must match x, and weight the last dimension")
    normed, r_out = np.empty_like(x), np.empty_like(x)
    lib().sor_add_rms_norm(_p(x), _p(r), None if w is None else _p(w), _p(normed), _p(r_out), x.size // dim, dim,
                           np.float32(eps))
    return normed, r_out


def layer_norm(x, weight, bias, eps: float) -> np.ndarray:
    """layernorm.rs:17-69 over the last axis; weight / bias may be None."""
    x = _f32(x)
    w = None if weight is None else _f32(weight)
    b = None if bias is None else _f32(bias)
    n = x.shape[-1]
    out = np.empty_like(x)
    lib().sor_layer_norm(_p(x), None if w is None else _p(w), None if b is None else _p(b), _p(out),
                         x.size // n, n, np.float32(eps))
    return out


def add_bias_last_dim(y, bias) -> np.ndarray:
    """common.rs:556-569: y + bias broadcast over the last dimension."""
    y, b = _f32(y), _f32(bias)
    if y.ndim == 0:
        raise ValueError("empty tensor")
    if b.size != y.shape[-1]:
        raise ValueError(f"bias length {b.size} does not match last dim {y.shape[-1]}")
    out = np.empty_like(y)
    lib().sor_add_bias_last_dim(_p(y), _p(b), _p(out), y.size, b.size)
    return out


def _binary(fn, a, b):
    a, b = _f32(a), _f32(b)
    n = max(a.size, b.size)
    out = np.empty(a.shape if a.size >= b.size else b.shape, np.float32)
    st = fn(_p(a), a.size, _p(b), b.size, _p(out))
    if st != OK:
        raise OracleError(st, "shape mismatch")
    return out.reshape(-1)[:n].reshape(out.shape)


def add(a, b) -> np.ndarray:
    return _binary(lib().sor_add, a, b)


def mul(a, b) -> np.ndarray:
    return _binary(lib().sor_mul, a, b)


def _unary(fn, x):
    x = _f32(x)
    out = np.empty_like(x)
    fn(_p(x), _p(out), x.size)
    return out


def silu(x) -> np.ndarray:
    return _unary(lib().sor_silu, x)


def gelu(x) -> np.ndarray:
    return _unary(lib().sor_gelu, x)


def gelu_erf(x) -> np.ndarray:
    return _unary(lib().sor_gelu_erf, x)


def swiglu(gate, up) -> np.ndarray:
    g, u = _f32(gate), _f32(up)
    out = np.empty_like(g)
    lib().sor_swiglu(_p(g), _p(u), _p(out), g.size)
    return out


def _positions(positions) -> np.ndarray:
    return np.ascontiguousarray(positions, dtype=np.int64)


def apply_rope(x, positions, base: float) -> np.ndarray:
    """rope::apply_rope (rope.rs:18-62); x is [B, H, S, D]."""
    x = _f32(x)
    pos = _positions(positions)
    B, H, S, D = x.shape
    out = np.empty_like(x)
    st = lib().sor_apply_rope(_p(x), _p(out), B, H, S, D, _p(pos), pos.size, np.float32(base))
    if st != OK:
        raise OracleError(st, "apply_rope")
    return out


def apply_rope_partial_scaled(x, positions, base: float, rotary_dim: int, pos_scale: float = 1.0,
                              interleaved: bool = False) -> np.ndarray:
    """rope::apply_rope_partial_scaled (rope.rs:83-136), or its interleaved-pair form."""
    x = _f32(x)
    pos = _positions(positions)
    B, H, S, D = x.shape
    out = np.empty_like(x)
    fn = lib().sor_apply_rope_interleaved if interleaved else lib().sor_apply_rope_partial_scaled
    st = fn(_p(x), _p(out), B, H, S, D, _p(pos), pos.size, np.float32(base), rotary_dim, np.float32(pos_scale))
    if st != OK:
        raise OracleError(st, "apply_rope")
    return out


def unpermute_qk_rows(rows: np.ndarray, n_head: int, head_dim: int) -> np.ndarray:
    """gguf_weights.rs:114-154 on a [n_head*head_dim, ...] array (any dtype)."""
    src = np.ascontiguousarray(rows)
    dst = np.empty_like(src)
    row_bytes = src.nbytes // src.shape[0]
    st = lib().sor_unpermute_qk_rows(_p(src), _p(dst), n_head, head_dim, row_bytes)
    if st != OK:
        raise OracleError(st, "unpermute_qk_rows")
    return dst


def row_bytes(dtype: int, hidden: int) -> int:
    return int(lib().sor_row_bytes(dtype, hidden))


def dequant(blocks: np.ndarray, dtype: int, numel: int) -> np.ndarray:
    """Tensor::to_f32_vec for a quantized tensor of `numel` elements (tensor.rs:362-398, 421-476)."""
    b = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.empty(numel, np.float32)
    fn = {Q4_0: (lib().sor_dequant_q4_0, 32), Q8_0: (lib().sor_dequant_q8_0, 32), Q4_K: (lib().sor_dequant_q4_k, 256),
          Q5_K: (lib().sor_dequant_q5_k, 256), Q6_K: (lib().sor_dequant_q6_k, 256)}[dtype]
    fn[0](_p(b), numel // fn[1], _p(out))
    return out


def embed_tokens(table: np.ndarray, dtype: int, vocab: int, hidden: int, ids) -> np.ndarray:
    """common::embed_tokens (common.rs:164-179); raises OracleError(ERANGE) on an id >= vocab."""
    t = np.ascontiguousarray(table).view(np.uint8).reshape(-1)
    idv = np.ascontiguousarray(ids, dtype=np.uint32)
    out = np.empty((idv.size, hidden), np.float32)
    st = lib().sor_embed_tokens(_p(t), dtype, vocab, hidden, _p(idv), idv.size, _p(out))
    if st != OK:
        raise OracleError(st, "embed_tokens")
    return out


def quantize_q8_0(x) -> np.ndarray:
    """quantize_q8_0_block (crates/sapient-backends/cpu/src/kernels/quant.rs:223-235), all blocks."""
    x = _f32(x).reshape(-1)
    out = np.empty(x.size // 32 * 34, np.uint8)
    lib().sor_quantize_q8_0(_p(x), x.size // 32, _p(out))
    return out


def transpose_heads(x, outer: int, inner: int, head_dim: int) -> np.ndarray:
    """resident.rs:420-458: [outer, inner, hd] -> [inner, outer, hd]; any 2- or
    4-byte element array (half tensors as uint16 bits) is moved as raw bytes."""
    x = np.ascontiguousarray(x)
    if x.size != outer * inner * head_dim or x.itemsize not in (2, 4):
        raise ValueError("x must hold outer * inner * head_dim 2- or 4-byte elements")
    out = np.empty((inner, outer, head_dim), x.dtype)
    lib().sor_transpose_heads(_p(x), _p(out), x.itemsize, outer, inner, head_dim)
    return out


def kv_append(src, cache: np.ndarray, cache_dtype: int, n_kv: int, seq: int, head_dim: int, max_seq: int,
              pos: int) -> None:
    """resident.rs:645-711, in place on `cache` ([n_kv, max_seq, hd]; float32, or
    uint16 bits for F16 / BF16; for Q8_0 uint8 [n_kv, max_seq, hd / 32 · 34], common.rs:449-508)."""
    src = _f32(src)
    row = head_dim // 32 * 34 if cache_dtype == Q8_0 else head_dim
    if src.size != n_kv * seq * head_dim or cache.size != n_kv * max_seq * row or not cache.flags.c_contiguous:
        raise ValueError("src / cache sizes do not match the layout")
    want = {F32: np.float32, Q8_0: np.uint8}.get(cache_dtype, np.uint16)
    if cache.dtype != want:
        raise ValueError("cache dtype does not match cache_dtype")
    st = lib().sor_kv_append(_p(src), _p(cache), cache_dtype, n_kv, seq, head_dim, max_seq, pos)
    if st != 0:
        raise OracleError(st, "kv_append")


def kv_cache_update(src, cache: np.ndarray, cache_dtype: int, n_kv: int, seq: int, head_dim: int, max_seq: int,
                    cur_len: int) -> int:
    """common.rs:355-434 (update_kv_cache) / :449-508 (update_kv_cache_q8), in place on
    `cache` (layouts as kv_append): appends src after cur_len rows per head, first
    sliding the window left by cur_len + seq - max_seq rows when that is positive.
    Returns the new length, min(cur_len + seq, max_seq)."""
    src = _f32(src)
    row = head_dim // 32 * 34 if cache_dtype == Q8_0 else head_dim
    if src.size != n_kv * seq * head_dim or cache.size != n_kv * max_seq * row or not cache.flags.c_contiguous:
        raise ValueError("src / cache sizes do not match the layout")
    want = {F32: np.float32, Q8_0: np.uint8}.get(cache_dtype, np.uint16)
    if cache.dtype != want:
        raise ValueError("cache dtype does not match cache_dtype")
    n = C.c_size_t(0)
    st = lib().sor_kv_cache_update(_p(src), _p(cache), cache_dtype, n_kv, seq, head_dim, max_seq, cur_len,
                                   C.byref(n))
    if st != 0:
        raise OracleError(st, "kv_cache_update")
    return n.value
