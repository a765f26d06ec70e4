"""ctypes binding of ``libsapient_hip.so`` (the C ABI in ``include/sapient_hip.h``).

Loading fails loudly if the library has not been built: there is no fallback
implementation of any op.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().with_name("libsapient_hip.so")

# status codes
OK, EINVAL, EHIP, ERANGE, ENODEV = 0, -1, -2, -3, -4
# dtype codes: GGUF tensor type ids
F32, F16, Q8_0, Q4_K, Q6_K, BF16 = 0, 1, 8, 12, 14, 30
ROPE_NEOX, ROPE_INTERLEAVED = 0, 1

# Every symbol the header declares, with its ctypes signature.
_vp, _i32, _i64, _f = C.c_void_p, C.c_int, C.c_int64, C.c_float
SIGNATURES = {
    "sph_abi_version": (_i32, []),
    "sph_status_string": (C.c_char_p, [_i32]),
    "sph_init": (_i32, [_vp]),
    "sph_rms_norm": (_i32, [_vp, _i32, _vp, _i32, _vp, _i32, _i64, _i64, _f, _vp]),
    "sph_add_rms_norm": (_i32, [_vp, _vp, _i32, _vp, _i32, _vp, _i32, _i64, _i64, _f, _vp]),
    "sph_layer_norm": (_i32, [_vp, _i32, _vp, _vp, _i32, _vp, _i32, _i64, _i64, _f, _vp]),
    "sph_add": (_i32, [_vp, _i64, _vp, _i64, _vp, _i32, _vp]),
    "sph_mul": (_i32, [_vp, _i64, _vp, _i64, _vp, _i32, _vp]),
    "sph_silu": (_i32, [_vp, _vp, _i32, _i64, _vp]),
    "sph_swiglu": (_i32, [_vp, _vp, _vp, _i32, _i64, _vp]),
    "sph_gelu_tanh": (_i32, [_vp, _vp, _i32, _i64, _vp]),
    "sph_gelu_erf": (_i32, [_vp, _vp, _i32, _i64, _vp]),
    "sph_add_bias": (_i32, [_vp, _vp, _i32, _vp, _i32, _i64, _i64, _vp]),
    "sph_rope": (_i32, [_vp, _i64, _vp, _i64, _i32, _i32, _vp, _i64, _i64, _i64, _i64, _f, _f, _vp]),
    "sph_embed": (_i32, [_vp, _i32, _i64, _i64, _vp, _i64, _vp, _vp, _vp]),
    "sph_rope_kv_append": (_i32, [_vp, _i64, _vp, _vp, _i64, _i32, _i32, _vp, _i64, _i64, _f, _f, _vp, _vp, _i32,
                                  _i64, _vp, _vp]),
    "sph_transpose_heads": (_i32, [_vp, _vp, _i32, _i64, _i64, _i64, _vp]),
    "sph_kv_append": (_i32, [_vp, _i32, _vp, _i32, _i64, _i64, _i64, _i64, _i64, _vp]),
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
