"""Device-resident op calls on torch tensors, through the C ABI.

torch supplies device memory and the current HIP stream; every op runs in the
HIP kernels of ``libsapient_hip.so``. Inputs must be contiguous device
tensors. Errors from the ABI raise :class:`SapientHipError`.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import torch

from . import _lib
from ._lib import check, lib

_DT = {torch.float32: _lib.F32, torch.float16: _lib.F16, torch.bfloat16: _lib.BF16}


def dtype_code(t: torch.dtype) -> int:
    try:
        return _DT[t]
    except KeyError:
        raise TypeError(f"unsupported dtype {t}") from None


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _dev(t: torch.Tensor, name: str) -> torch.Tensor:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    return t


def _out(out: Optional[torch.Tensor], shape, dtype: torch.dtype, device, name: str = "out") -> torch.Tensor:
    """A fresh output, or the caller's after checking it holds exactly what the kernel writes."""
    if out is None:
        return torch.empty(shape, dtype=dtype, device=device)
    _dev(out, name)
    numel = 1
    for d in shape:
        numel *= d
    if out.numel() != numel or out.dtype != dtype:
        raise ValueError(f"{name} must hold {numel} elements of {dtype}")
    return out


def init(device: Optional[torch.device] = None) -> None:
    """Per-device set-up (GELU tables); optional, done lazily otherwise."""
    with torch.cuda.device(device or torch.cuda.current_device()):
        check(lib().sph_init(torch.cuda.current_stream().cuda_stream), "init")


def rms_norm(x: torch.Tensor, weight: Optional[torch.Tensor], eps: float,
             out: Optional[torch.Tensor] = None, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """RMSNorm over the last dim (layernorm.rs:75-106). out_dtype: f32 (the
    reference's output type) or x's dtype; defaults to x's dtype."""
    _dev(x, "x")
    dim = x.shape[-1] if x.dim() else 1
    rows = x.numel() // dim if dim else 0
    od = out_dtype or (out.dtype if out is not None else x.dtype)
    out = _out(out, x.shape, od, x.device)
    w = _vec(weight, dim, "weight")
    check(lib().sph_rms_norm(x.data_ptr(), dtype_code(x.dtype),
                             None if w is None else w.data_ptr(), dtype_code(w.dtype) if w is not None else 0,
                             out.data_ptr(), dtype_code(out.dtype), rows, dim, float(eps), _stream(x)),
          "rms_norm")
    return out


def _vec(t: Optional[torch.Tensor], n: int, name: str) -> Optional[torch.Tensor]:
    if t is None:
        return None
    _dev(t, name)
    if t.numel() != n:
        raise ValueError(f"{name} length {t.numel()} does not match last dim {n}")
    return t


def layer_norm(x: torch.Tensor, weight: Optional[torch.Tensor], bias: Optional[torch.Tensor], eps: float,
               out: Optional[torch.Tensor] = None, out_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """LayerNorm over the last dim (layernorm.rs:17-69, axis -1; common.rs:575-577).
    weight and bias are optional and share one dtype (f32 or x's)."""
    _dev(x, "x")
    dim = x.shape[-1] if x.dim() else 1
    rows = x.numel() // dim if dim else 0
    od = out_dtype or (out.dtype if out is not None else x.dtype)
    out = _out(out, x.shape, od, x.device)
    w = _vec(weight, dim, "weight")
    b = _vec(bias, dim, "bias")
    if w is not None and b is not None and w.dtype != b.dtype:
        raise ValueError("weight and bias must share dtype")
    wb = w if w is not None else b
    check(lib().sph_layer_norm(x.data_ptr(), dtype_code(x.dtype), None if w is None else w.data_ptr(),
                               None if b is None else b.data_ptr(), dtype_code(wb.dtype) if wb is not None else 0,
                               out.data_ptr(), dtype_code(out.dtype), rows, dim, float(eps), _stream(x)),
          "layer_norm")
    return out


def add_rms_norm(x: torch.Tensor, residual: torch.Tensor, weight: Optional[torch.Tensor], eps: float,
                 out: Optional[torch.Tensor] = None,
                 out_dtype: Optional[torch.dtype] = None,
                 sum_out: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Fused add (llama.rs:508) + rms_norm (llama.rs:515). `residual` is
    updated in place with x + residual, or, given `sum_out`, left as it is while
    the sum goes to `sum_out` (as the trait's add returns a new tensor); returns
    (normed, sum)."""
    _dev(x, "x")
    _dev(residual, "residual")
    if residual.shape != x.shape or residual.dtype != x.dtype:
        raise ValueError("x and residual must share shape and dtype")
    if sum_out is not None:
        _dev(sum_out, "sum_out")
        if sum_out.shape != x.shape or sum_out.dtype != x.dtype:
            raise ValueError("sum_out must share x's shape and dtype")
    dim = x.shape[-1]
    rows = x.numel() // dim if dim else 0
    od = out_dtype or (out.dtype if out is not None else x.dtype)
    out = _out(out, x.shape, od, x.device)
    w = _vec(weight, dim, "weight")
    wp, wd = (None, 0) if w is None else (w.data_ptr(), dtype_code(w.dtype))
    if sum_out is None:
        check(lib().sph_add_rms_norm(x.data_ptr(), residual.data_ptr(), dtype_code(x.dtype), wp, wd,
                                     out.data_ptr(), dtype_code(out.dtype), rows, dim, float(eps), _stream(x)),
              "add_rms_norm")
        return out, residual
    check(lib().sph_add_rms_norm_to(x.data_ptr(), residual.data_ptr(), sum_out.data_ptr(), dtype_code(x.dtype), wp,
                                    wd, out.data_ptr(), dtype_code(out.dtype), rows, dim, float(eps), _stream(x)),
          "add_rms_norm")
    return out, sum_out


def _binary(fn, name, a, b, out):
    _dev(a, "a")
    _dev(b, "b")
    if a.dtype != b.dtype:
        raise ValueError("operands must share dtype")
    big = a if a.numel() >= b.numel() else b
    out = _out(out, big.shape, a.dtype, a.device)
    check(fn(a.data_ptr(), a.numel(), b.data_ptr(), b.numel(), out.data_ptr(), dtype_code(a.dtype), _stream(a)), name)
    return out


def add(a: torch.Tensor, b: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """a + b with the reference's length-1 broadcast (elementwise.rs:27-63)."""
    return _binary(lib().sph_add, "add", a, b, out)


def mul(a: torch.Tensor, b: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """a * b with the reference's length-1 broadcast (elementwise.rs:27-57, :67-69)."""
    return _binary(lib().sph_mul, "mul", a, b, out)


def silu(x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    _dev(x, "x")
    out = _out(out, x.shape, x.dtype, x.device)
    check(lib().sph_silu(x.data_ptr(), out.data_ptr(), dtype_code(x.dtype), x.numel(), _stream(x)), "silu")
    return out


def swiglu(gate: torch.Tensor, up: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """silu(gate) * up, fused (llama.rs:531-532)."""
    _dev(gate, "gate")
    _dev(up, "up")
    if gate.shape != up.shape or gate.dtype != up.dtype:
        raise ValueError("gate and up must share shape and dtype")
    out = _out(out, gate.shape, gate.dtype, gate.device)
    check(lib().sph_swiglu(gate.data_ptr(), up.data_ptr(), out.data_ptr(), dtype_code(gate.dtype), gate.numel(),
                           _stream(gate)), "swiglu")
    return out


def gelu_tanh(x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """GELU tanh form (elementwise.rs:120-127), bit-exact with the reference."""
    _dev(x, "x")
    out = _out(out, x.shape, x.dtype, x.device)
    check(lib().sph_gelu_tanh(x.data_ptr(), out.data_ptr(), dtype_code(x.dtype), x.numel(), _stream(x)), "gelu")
    return out


def gelu_erf(x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """GELU erf form (elementwise.rs:135-138, :163-174), bit-exact with the reference."""
    _dev(x, "x")
    out = _out(out, x.shape, x.dtype, x.device)
    check(lib().sph_gelu_erf(x.data_ptr(), out.data_ptr(), dtype_code(x.dtype), x.numel(), _stream(x)), "gelu_erf")
    return out


def add_bias(y: torch.Tensor, bias: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y + bias over the last dim (common.rs:556-569); bias may be f32 or a half type."""
    _dev(y, "y")
    if y.dim() == 0:
        raise ValueError("empty tensor")
    n = y.shape[-1]
    _dev(bias, "bias")
    if bias.numel() != n:
        raise ValueError(f"bias length {bias.numel()} does not match last dim {n}")
    out = _out(out, y.shape, y.dtype, y.device)
    check(lib().sph_add_bias(y.data_ptr(), bias.data_ptr(), dtype_code(bias.dtype), out.data_ptr(),
                             dtype_code(y.dtype), y.numel(), n, _stream(y)), "add_bias")
    return out


def rope_(q: torch.Tensor, k: Optional[torch.Tensor], positions: torch.Tensor, base: float,
          rotary_dim: Optional[int] = None, pos_scale: float = 1.0, interleaved: bool = False) -> None:
    """RoPE in place on q [B, Hq, S, D] and optionally k [B, Hk, S, D]
    (rope.rs:18-62 / :83-136). positions: int32 device tensor [S]."""
    _dev(q, "q")
    if q.dim() != 4:
        raise ValueError("q must be [batch, heads, seq, head_dim]")
    B, Hq, S, D = q.shape
    Hk = 0
    if k is not None:
        _dev(k, "k")
        if k.dim() != 4 or k.shape[0] != B or k.shape[2] != S or k.shape[3] != D or k.dtype != q.dtype:
            raise ValueError("k must be [batch, kv_heads, seq, head_dim] like q")
        Hk = k.shape[1]
    _dev(positions, "positions")
    if positions.dtype != torch.int32 or positions.numel() != S:
        raise ValueError("positions must be int32 with seq_len entries")
    rd = D if rotary_dim is None else rotary_dim
    layout = _lib.ROPE_INTERLEAVED if interleaved else _lib.ROPE_NEOX
    check(lib().sph_rope(q.data_ptr(), Hq, None if k is None else k.data_ptr(), Hk, dtype_code(q.dtype), layout,
                         positions.data_ptr(), B, S, D, rd, float(base), float(pos_scale), _stream(q)), "rope")


def rope_table(positions, rotary_dim: int, base: float, pos_scale: float = 1.0, n: Optional[int] = None):
    """Host cos / sin tables [n, rotary_dim / 2] (float32 numpy) of the RoPE angles of `positions` (a
    sequence of ints, row r for positions[r]) or, with positions None, of 0 .. n - 1 — the layout of
    rope_cos_sin_cache (rope.rs:140-153), evaluated by the library with the host libm (rope.rs:48-50)."""
    import numpy as np
    if positions is None:
        if n is None:
            raise ValueError("give positions or n")
        pos, count = None, int(n)
    else:
        pos = np.ascontiguousarray(positions, dtype=np.int64)
        count = pos.size
    if rotary_dim <= 0 or rotary_dim % 2:
        raise ValueError("rotary_dim must be even and positive")
    cs = np.empty((count, rotary_dim // 2), np.float32)
    sn = np.empty((count, rotary_dim // 2), np.float32)
    check(lib().sph_rope_table(None if pos is None else pos.ctypes.data, count, rotary_dim, float(base),
                               float(pos_scale), cs.ctypes.data, sn.ctypes.data), "rope_table")
    return cs, sn


def rope_cached_(q: torch.Tensor, k: Optional[torch.Tensor], cos_table: torch.Tensor, sin_table: torch.Tensor,
                 positions: Optional[torch.Tensor] = None, rotary_dim: Optional[int] = None,
                 interleaved: bool = False, bad_pos_flag: Optional[torch.Tensor] = None) -> None:
    """RoPE in place on q [B, Hq, S, D] (and k) with the angles read from device f32 tables
    [rows, rotary_dim / 2]: token s uses row positions[s] (int32 device tensor [S]), or row s when
    positions is None."""
    _dev(q, "q")
    if q.dim() != 4:
        raise ValueError("q must be [batch, heads, seq, head_dim]")
    B, Hq, S, D = q.shape
    Hk = 0
    if k is not None:
        _dev(k, "k")
        if k.dim() != 4 or k.shape[0] != B or k.shape[2] != S or k.shape[3] != D or k.dtype != q.dtype:
            raise ValueError("k must be [batch, kv_heads, seq, head_dim] like q")
        Hk = k.shape[1]
    rd = D if rotary_dim is None else rotary_dim
    for t, name in ((cos_table, "cos_table"), (sin_table, "sin_table")):
        _dev(t, name)
        if t.dtype != torch.float32 or t.dim() != 2 or t.shape[1] != rd // 2:
            raise ValueError(f"{name} must be f32 [rows, rotary_dim / 2]")
    if cos_table.shape != sin_table.shape:
        raise ValueError("cos_table and sin_table must have the same shape")
    if positions is not None:
        _dev(positions, "positions")
        if positions.dtype != torch.int32 or positions.numel() != S:
            raise ValueError("positions must be int32 with seq_len entries")
    flag = None
    if bad_pos_flag is not None:
        flag = _dev(bad_pos_flag, "bad_pos_flag")
        if flag.dtype != torch.int32 or flag.numel() < 1:
            raise ValueError("bad_pos_flag must be an int32 device tensor")
    layout = _lib.ROPE_INTERLEAVED if interleaved else _lib.ROPE_NEOX
    check(lib().sph_rope_cached(q.data_ptr(), Hq, None if k is None else k.data_ptr(), Hk, dtype_code(q.dtype),
                                layout, cos_table.data_ptr(), sin_table.data_ptr(), cos_table.shape[0],
                                None if positions is None else positions.data_ptr(), B, S, D, rd,
                                None if flag is None else flag.data_ptr(), _stream(q)), "rope_cached")


def rope_host_positions_(q: torch.Tensor, k: Optional[torch.Tensor], positions, base: float,
                         rotary_dim: Optional[int] = None, pos_scale: float = 1.0, interleaved: bool = False) -> None:
    """The trait path's RoPE (apply_rope_positions, backend.rs:84): positions on the host, angles evaluated
    on the host for exactly those positions (rope_table), uploaded, and applied by rope_cached_."""
    rd = q.shape[-1] if rotary_dim is None else rotary_dim
    cs, sn = rope_table(positions, rd, base, pos_scale)
    cs_d = torch.from_numpy(cs).to(q.device, non_blocking=False)
    sn_d = torch.from_numpy(sn).to(q.device, non_blocking=False)
    rope_cached_(q, k, cs_d, sn_d, None, rd, interleaved)


# Bytes per row as (bytes per block, elements per block) of each table type
# (crates/sapient-core/src/dtype.rs:136-145).
_ROW_BYTES = {_lib.F32: (4, 1), _lib.F16: (2, 1), _lib.BF16: (2, 1), _lib.Q4_0: (18, 32), _lib.Q8_0: (34, 32),
              _lib.Q4_K: (144, 256), _lib.Q5_K: (176, 256), _lib.Q6_K: (210, 256)}


def embed(table: torch.Tensor, table_dtype: int, vocab: int, hidden: int, ids: torch.Tensor,
          out: Optional[torch.Tensor] = None, bad_id_flag: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Row gather + dequant of a raw GGUF table (common.rs:164-217) into f32
    [n_ids, hidden]. `table` holds the raw tensor bytes (any dtype, contiguous);
    ids: int32/uint32 device tensor (ids are read as uint32)."""
    _dev(table, "table")
    _dev(ids, "ids")
    if ids.dtype not in (torch.int32, torch.uint32):
        raise ValueError("ids must be 32-bit")
    n = ids.numel()
    if table_dtype not in _ROW_BYTES or hidden < 0 or vocab < 0:
        raise ValueError("unsupported table dtype or negative size")
    num, den = _ROW_BYTES[table_dtype]
    if hidden % den == 0 and table.numel() * table.element_size() < vocab * (hidden // den) * num:
        raise ValueError("table holds fewer than vocab rows")
    out = _out(out, (n, hidden), torch.float32, ids.device)
    flag = None
    if bad_id_flag is not None:
        flag = _dev(bad_id_flag, "bad_id_flag")
        if flag.dtype != torch.int32 or flag.numel() < 1:
            raise ValueError("bad_id_flag must be an int32 device tensor")
    check(lib().sph_embed(table.data_ptr(), table_dtype, vocab, hidden, ids.data_ptr(), n, out.data_ptr(),
                          None if flag is None else flag.data_ptr(), _stream(ids)), "embed")
    return out


def transpose_heads(x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """[outer, inner, head_dim] -> [inner, outer, head_dim] (resident.rs:420-458), bit for bit."""
    _dev(x, "x")
    if x.dim() != 3:
        raise ValueError("x must be [outer, inner, head_dim]")
    outer, inner, hd = x.shape
    out = _out(out, (inner, outer, hd), x.dtype, x.device)
    if out.data_ptr() == x.data_ptr() and x.numel():
        raise ValueError("out must not alias x")
    check(lib().sph_transpose_heads(x.data_ptr(), out.data_ptr(), dtype_code(x.dtype), outer, inner, hd, _stream(x)),
          "transpose_heads")
    return out


def kv_append(src: torch.Tensor, cache: torch.Tensor, pos: int) -> None:
    """Write src [n_kv, seq, head_dim] into cache [n_kv, max_seq, head_dim] at
    positions pos..pos+seq, converted to the cache's dtype (resident.rs:645-711).
    A uint8 cache [n_kv, max_seq, head_dim / 32 * 34] is a Q8_0 cache, quantized
    on append (common.rs:336-348, :449-508)."""
    _dev(src, "src")
    _dev(cache, "cache")
    q8 = cache.dtype == torch.uint8
    if src.dim() != 3 or cache.dim() != 3 or src.shape[0] != cache.shape[0]:
        raise ValueError("src must be [n_kv, seq, head_dim] and cache [n_kv, max_seq, row]")
    n_kv, seq, hd = src.shape
    if cache.shape[2] != (hd // 32 * 34 if q8 else hd) or (q8 and hd % 32):
        raise ValueError("cache rows must hold head_dim elements (Q8_0: head_dim / 32 blocks of 34 bytes)")
    max_seq = cache.shape[1]
    cdt = _lib.Q8_0 if q8 else dtype_code(cache.dtype)
    check(lib().sph_kv_append(src.data_ptr(), dtype_code(src.dtype), cache.data_ptr(), cdt,
                              n_kv, seq, hd, max_seq, int(pos), _stream(src)), "kv_append")


def kv_cache_update(src: torch.Tensor, cache: torch.Tensor, cur_len: int) -> int:
    """Append src [n_kv, seq, head_dim] after the cur_len valid rows of each head
    of cache [n_kv, max_seq, row], sliding the window left first when the rows
    would not fit, and return the new valid length min(cur_len + seq, max_seq):
    common::update_kv_cache / update_kv_cache_q8 (common.rs:355-434, :449-508).
    Cache dtypes as kv_append (a uint8 cache is Q8_0)."""
    _dev(src, "src")
    _dev(cache, "cache")
    q8 = cache.dtype == torch.uint8
    if src.dim() != 3 or cache.dim() != 3 or src.shape[0] != cache.shape[0]:
        raise ValueError("src must be [n_kv, seq, head_dim] and cache [n_kv, max_seq, row]")
    n_kv, seq, hd = src.shape
    if cache.shape[2] != (hd // 32 * 34 if q8 else hd) or (q8 and hd % 32):
        raise ValueError("cache rows must hold head_dim elements (Q8_0: head_dim / 32 blocks of 34 bytes)")
    max_seq = cache.shape[1]
    cdt = _lib.Q8_0 if q8 else dtype_code(cache.dtype)
    n = ctypes.c_int64(0)
    check(lib().sph_kv_cache_update(src.data_ptr(), dtype_code(src.dtype), cache.data_ptr(), cdt, n_kv, seq, hd,
                                    max_seq, int(cur_len), ctypes.addressof(n), _stream(src)), "kv_cache_update")
    return n.value


def kv_cache_update_into(src: torch.Tensor, cache: torch.Tensor, out: torch.Tensor, cur_len: int) -> int:
    """kv_cache_update into a second cache: `out` (cache's shape and dtype) receives rows [0, new_len) of the
    updated cache — cache's kept rows moved once, then src — and `cache` is only read. The caller then uses
    `out` as its cache (common.rs:355-434, :449-508 take the cache as &mut Tensor). Returns new_len."""
    _dev(src, "src")
    _dev(cache, "cache")
    _dev(out, "out")
    q8 = cache.dtype == torch.uint8
    if src.dim() != 3 or cache.dim() != 3 or src.shape[0] != cache.shape[0]:
        raise ValueError("src must be [n_kv, seq, head_dim] and cache [n_kv, max_seq, row]")
    if out.shape != cache.shape or out.dtype != cache.dtype:
        raise ValueError("out must have the cache's shape and dtype")
    n_kv, seq, hd = src.shape
    if cache.shape[2] != (hd // 32 * 34 if q8 else hd) or (q8 and hd % 32):
        raise ValueError("cache rows must hold head_dim elements (Q8_0: head_dim / 32 blocks of 34 bytes)")
    max_seq = cache.shape[1]
    cdt = _lib.Q8_0 if q8 else dtype_code(cache.dtype)
    n = ctypes.c_int64(0)
    check(lib().sph_kv_cache_update_into(src.data_ptr(), dtype_code(src.dtype), cache.data_ptr(), out.data_ptr(),
                                         cdt, n_kv, seq, hd, max_seq, int(cur_len), ctypes.addressof(n),
                                         _stream(src)), "kv_cache_update_into")
    return n.value


def _rope_kv_args(Hq, Hkv, S, D, positions, kcache, vcache, bad_pos_flag, bq, bk, bv):
    """Checks shared by the fused decode steps; returns (flag, biases, bias dtype code)."""
    for t, n in ((kcache, "kcache"), (vcache, "vcache"), (positions, "positions")):
        _dev(t, n)
    if kcache.shape != vcache.shape or kcache.dim() != 3 or kcache.shape[0] != Hkv or kcache.shape[2] != D \
            or kcache.dtype != vcache.dtype:
        raise ValueError("caches must be [Hkv, max_seq, D] of one dtype")
    if positions.dtype != torch.int32 or positions.numel() != S:
        raise ValueError("positions must be int32 with seq entries")
    flag = None
    if bad_pos_flag is not None:
        flag = _dev(bad_pos_flag, "bad_pos_flag")
        if flag.dtype != torch.int32 or flag.numel() < 1:
            raise ValueError("bad_pos_flag must be an int32 device tensor")
    biases = [_vec(bq, Hq * D, "bq"), _vec(bk, Hkv * D, "bk"), _vec(bv, Hkv * D, "bv")]
    bdt = {b.dtype for b in biases if b is not None}
    if len(bdt) > 1:
        raise ValueError("biases must share dtype")
    bias_code = dtype_code(bdt.pop()) if bdt else 0
    return flag, [None if b is None else b.data_ptr() for b in biases], bias_code


def rope_kv_append(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, positions: torch.Tensor, base: float,
                   kcache: torch.Tensor, vcache: torch.Tensor, pos_scale: float = 1.0, interleaved: bool = False,
                   bad_pos_flag: Optional[torch.Tensor] = None, bq: Optional[torch.Tensor] = None,
                   bk: Optional[torch.Tensor] = None, bv: Optional[torch.Tensor] = None) -> None:
    """Fused decode step: optional q/k/v biases, RoPE on q in place; rotated k and v written to
    the caches at rows positions[s] (wgpu_engine.rs:397-432). q [Hq, S, D], k/v [Hkv, S, D],
    caches [Hkv, max_seq, D], biases [Hq·D] / [Hkv·D] of one dtype."""
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _dev(t, n)
    if q.dim() != 3 or k.dim() != 3 or k.shape != v.shape or q.shape[1:] != k.shape[1:]:
        raise ValueError("q must be [Hq, S, D] and k, v [Hkv, S, D]")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("q, k and v must share dtype")
    Hq, S, D = q.shape
    Hkv = k.shape[0]
    flag, biases, bias_code = _rope_kv_args(Hq, Hkv, S, D, positions, kcache, vcache, bad_pos_flag, bq, bk, bv)
    layout = _lib.ROPE_INTERLEAVED if interleaved else _lib.ROPE_NEOX
    check(lib().sph_rope_kv_append(q.data_ptr(), Hq, k.data_ptr(), v.data_ptr(), Hkv, dtype_code(q.dtype), layout,
                                   positions.data_ptr(), S, D, float(base), float(pos_scale), kcache.data_ptr(),
                                   vcache.data_ptr(), dtype_code(kcache.dtype), kcache.shape[1], *biases, bias_code,
                                   None if flag is None else flag.data_ptr(), _stream(q)), "rope_kv_append")


def rope_kv_append_tokens(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, positions: torch.Tensor, base: float,
                          kcache: torch.Tensor, vcache: torch.Tensor, pos_scale: float = 1.0,
                          interleaved: bool = False, bad_pos_flag: Optional[torch.Tensor] = None,
                          bq: Optional[torch.Tensor] = None, bk: Optional[torch.Tensor] = None,
                          bv: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The fused step on a chunk in the projections' layout: q [S, Hq, D], k/v [S, Hkv, D] token-major
    (read only); returns the rotated q heads-major [Hq, S, D] (wgpu_engine.rs:525-573 without the
    transposes); k and v rows go to the caches as in rope_kv_append."""
    for t, n in ((q, "q"), (k, "k"), (v, "v")):
        _dev(t, n)
    if q.dim() != 3 or k.dim() != 3 or k.shape != v.shape or q.shape[0] != k.shape[0] or q.shape[2] != k.shape[2]:
        raise ValueError("q must be [S, Hq, D] and k, v [S, Hkv, D]")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("q, k and v must share dtype")
    S, Hq, D = q.shape
    Hkv = k.shape[1]
    flag, biases, bias_code = _rope_kv_args(Hq, Hkv, S, D, positions, kcache, vcache, bad_pos_flag, bq, bk, bv)
    q_out = _out(out, (Hq, S, D), q.dtype, q.device)
    layout = _lib.ROPE_INTERLEAVED if interleaved else _lib.ROPE_NEOX
    check(lib().sph_rope_kv_append_tokens(q.data_ptr(), q_out.data_ptr(), Hq, k.data_ptr(), v.data_ptr(), Hkv,
                                          dtype_code(q.dtype), layout, positions.data_ptr(), S, D, float(base),
                                          float(pos_scale), kcache.data_ptr(), vcache.data_ptr(),
                                          dtype_code(kcache.dtype), kcache.shape[1], *biases, bias_code,
                                          None if flag is None else flag.data_ptr(), _stream(q)),
          "rope_kv_append_tokens")
    return q_out
