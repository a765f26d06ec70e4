"""ctypes binding of ``libsapient_hip.so`` (the C ABI in ``include/sapient_hip.h``
and the decode engine of ``include/sapient_hip_engine.h``).

Loading fails loudly if the library has not been built: there is no fallback
implementation of any op.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().with_name("libsapient_hip.so")

# status codes
OK, EINVAL, EHIP, ERANGE, ENODEV, ESTATE = 0, -1, -2, -3, -4, -5
# dtype codes: GGUF tensor type ids
F32, F16, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K, BF16 = 0, 1, 2, 8, 12, 13, 14, 30
ROPE_NEOX, ROPE_INTERLEAVED = 0, 1

# Every symbol the headers declare, with its ctypes signature.
_vp, _i32, _i64, _f = C.c_void_p, C.c_int, C.c_int64, C.c_float


class EngineConfig(C.Structure):
    """sph_engine_config."""
    _fields_ = [("hidden", C.c_int64), ("n_heads", C.c_int64), ("n_kv_heads", C.c_int64), ("head_dim", C.c_int64),
                ("intermediate", C.c_int64), ("n_layers", C.c_int64), ("max_seq", C.c_int64),
                ("max_chunk", C.c_int64), ("rms_eps", C.c_float), ("rope_theta", C.c_float),
                ("rope_layout", C.c_int), ("kv_dtype", C.c_int), ("bias_dtype", C.c_int)]


class EngineLayer(C.Structure):
    """sph_engine_layer: device pointers."""
    _fields_ = [("input_ln", C.c_void_p), ("post_ln", C.c_void_p), ("bq", C.c_void_p), ("bk", C.c_void_p),
                ("bv", C.c_void_p), ("bo", C.c_void_p)]


PROJ_Q, PROJ_K, PROJ_V, PROJ_O, PROJ_GATE, PROJ_UP, PROJ_DOWN = range(7)
# int (*)(void* user, int layer, int which, const float* in, float* out, int64_t rows, void* stream)
PROJECT_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_int64, C.c_void_p)
# int (*)(void* user, int layer, const float* q, const void* kc, const void* vc, int kv_dtype,
#         const int32_t* positions, int64_t n_tok, int64_t max_seq, float* out, void* stream)
ATTEND_FN = C.CFUNCTYPE(C.c_int, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p,
                        C.c_int64, C.c_int64, C.c_void_p, C.c_void_p)
SIGNATURES = {
    "sph_abi_version": (_i32, []),
    "sph_status_string": (C.c_char_p, [_i32]),
    "sph_init": (_i32, [_vp]),
    "sph_rms_norm": (_i32, [_vp, _i32, _vp, _i32, _vp, _i32, _i64, _i64, _f, _vp]),
    "sph_add_rms_norm": (_i32, [_vp, _vp, _i32, _vp, _i32, _vp, _i32, _i64, _i64, _f, _vp]),
    "sph_add_rms_norm_to": (_i32, [_vp, _vp, _vp, _i32, _vp, _i32, _vp, _i32, _i64, _i64, _f, _vp]),
    "sph_layer_norm": (_i32, [_vp, _i32, _vp, _vp, _i32, _vp, _i32, _i64, _i64, _f, _vp]),
    "sph_add": (_i32, [_vp, _i64, _vp, _i64, _vp, _i32, _vp]),
    "sph_mul": (_i32, [_vp, _i64, _vp, _i64, _vp, _i32, _vp]),
    "sph_silu": (_i32, [_vp, _vp, _i32, _i64, _vp]),
    "sph_swiglu": (_i32, [_vp, _vp, _vp, _i32, _i64, _vp]),
    "sph_gelu_tanh": (_i32, [_vp, _vp, _i32, _i64, _vp]),
    "sph_gelu_erf": (_i32, [_vp, _vp, _i32, _i64, _vp]),
    "sph_add_bias": (_i32, [_vp, _vp, _i32, _vp, _i32, _i64, _i64, _vp]),
    "sph_rope": (_i32, [_vp, _i64, _vp, _i64, _i32, _i32, _vp, _i64, _i64, _i64, _i64, _f, _f, _vp]),
    "sph_rope_cached": (_i32, [_vp, _i64, _vp, _i64, _i32, _i32, _vp, _vp, _i64, _vp, _i64, _i64, _i64, _i64, _vp,
                               _vp]),
    "sph_rope_table": (_i32, [_vp, _i64, _i64, _f, _f, _vp, _vp]),
    "sph_embed": (_i32, [_vp, _i32, _i64, _i64, _vp, _i64, _vp, _vp, _vp]),
    "sph_rope_kv_append": (_i32, [_vp, _i64, _vp, _vp, _i64, _i32, _i32, _vp, _i64, _i64, _f, _f, _vp, _vp, _i32,
                                  _i64, _vp, _vp, _vp, _i32, _vp, _vp]),
    "sph_rope_kv_append_tokens": (_i32, [_vp, _vp, _i64, _vp, _vp, _i64, _i32, _i32, _vp, _i64, _i64, _f, _f, _vp,
                                         _vp, _i32, _i64, _vp, _vp, _vp, _i32, _vp, _vp]),
    "sph_transpose_heads": (_i32, [_vp, _vp, _i32, _i64, _i64, _i64, _vp]),
    "sph_kv_append": (_i32, [_vp, _i32, _vp, _i32, _i64, _i64, _i64, _i64, _i64, _vp]),
    "sph_kv_cache_update": (_i32, [_vp, _i32, _vp, _i32, _i64, _i64, _i64, _i64, _i64, _vp, _vp]),
    "sph_kv_cache_update_into": (_i32, [_vp, _i32, _vp, _vp, _i32, _i64, _i64, _i64, _i64, _i64, _vp, _vp]),
    # sapient_hip_engine.h
    "sph_engine_create": (_i32, [C.POINTER(EngineConfig), _vp, _i32, _i64, C.POINTER(EngineLayer), _vp, PROJECT_FN,
                                 ATTEND_FN, _vp, C.POINTER(_vp)]),
    "sph_engine_destroy": (None, [_vp]),
    "sph_engine_forward_token": (_i32, [_vp, C.c_uint32, C.POINTER(_vp)]),
    "sph_engine_forward_chunk": (_i32, [_vp, _vp, _i64, C.POINTER(_vp)]),
    "sph_engine_use_graph": (_i32, [_vp, _i32]),
    "sph_engine_reset": (_i32, [_vp]),
    "sph_engine_position": (_i64, [_vp]),
    "sph_engine_stream": (_vp, [_vp]),
    "sph_engine_kcache": (_vp, [_vp, _i32]),
    "sph_engine_vcache": (_vp, [_vp, _i32]),
}

_lib = None


class SapientHipError(RuntimeError):
    """A non-zero status from the C ABI."""

    def __init__(self, status: int, op: str):
        msg = lib().sph_status_string(status).decode() if _lib is not None else str(status)
        super().__init__(f"{op}: {msg} (status {status})")
        self.status = status


def lib() -> C.CDLL:
    """Load the shared library once (import torch first so both share one HIP runtime)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH.name} is not built; run `python -m sapient_amd.build` (hipcc, gfx950)")
        L = C.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(status: int, op: str) -> None:
    if status != OK:
        raise SapientHipError(status, op)
