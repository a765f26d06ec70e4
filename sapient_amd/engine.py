"""The device-resident decode engine (``include/sapient_hip_engine.h``) from Python.

A thin ctypes wrapper: torch supplies the weight tensors (device memory the
caller keeps alive), the engine owns its activations and KV caches. Callbacks
for the projections and attention are Python callables ``project(layer, which,
in_ptr, out_ptr, rows, stream)`` and ``attend(layer, q_ptr, kcache_ptr,
vcache_ptr, kv_dtype, positions_ptr, n_tok, max_seq, out_ptr, stream)``; they
must enqueue their work on ``stream`` and return 0. ``None`` skips the stage.
"""
from __future__ import annotations

import ctypes as C
from typing import Callable, Optional, Sequence

import torch

from . import _lib
from ._lib import check, lib


class _DevArray:
    """A raw device pointer seen by torch through the CUDA array interface (no copy)."""

    def __init__(self, ptr: int, shape, typestr: str):
        self.__cuda_array_interface__ = {"shape": tuple(shape), "typestr": typestr, "data": (ptr, False),
                                         "version": 2, "strides": None}


_TYPESTR = {_lib.F32: "<f4", _lib.F16: "<f2", _lib.BF16: "<u2"}


class Engine:
    def __init__(self, cfg: _lib.EngineConfig, embed_table: torch.Tensor, embed_dtype: int, vocab: int,
                 layers: Sequence[dict], final_norm: torch.Tensor,
                 project: Optional[Callable] = None, attend: Optional[Callable] = None):
        """layers: dicts with device tensors input_ln, post_ln and optional bq, bk, bv, bo."""
        self.cfg = cfg
        self._keep = [embed_table, final_norm] + [t for L in layers for t in L.values() if t is not None]
        arr = (_lib.EngineLayer * len(layers))()
        for i, L in enumerate(layers):
            ptr = lambda name: None if L.get(name) is None else L[name].data_ptr()
            arr[i] = _lib.EngineLayer(ptr("input_ln"), ptr("post_ln"), ptr("bq"), ptr("bk"), ptr("bv"), ptr("bo"))
        self._project = _lib.PROJECT_FN(self._wrap(project)) if project else _lib.PROJECT_FN()
        self._attend = _lib.ATTEND_FN(self._wrap(attend)) if attend else _lib.ATTEND_FN()
        handle = C.c_void_p()
        check(lib().sph_engine_create(C.byref(cfg), embed_table.data_ptr(), embed_dtype, vocab, arr,
                                      final_norm.data_ptr(), self._project, self._attend, None, C.byref(handle)),
              "engine_create")
        self.handle = handle
        self.stream = torch.cuda.ExternalStream(lib().sph_engine_stream(handle))

    @staticmethod
    def _wrap(fn):
        def call(_user, *args):
            try:
                return int(fn(*args) or 0)
            except Exception:  # a Python error must not unwind through C
                return _lib.EHIP
        return call

    def close(self) -> None:
        if self.handle:
            lib().sph_engine_destroy(self.handle)
            self.handle = None

    def __del__(self):
        self.close()

    def _hidden(self, ptr: C.c_void_p) -> torch.Tensor:
        # torch's current stream waits for the engine's work before using the result.
        torch.cuda.current_stream().wait_stream(self.stream)
        return torch.as_tensor(_DevArray(ptr.value, (self.cfg.hidden,), "<f4"), device="cuda")

    def forward_token(self, tok: int) -> torch.Tensor:
        """Device view of the final hidden state, valid until the next call. The work runs on
        self.stream; torch's current stream is made to wait for it."""
        out = C.c_void_p()
        self.stream.wait_stream(torch.cuda.current_stream())  # earlier readers of the buffers finish first
        check(lib().sph_engine_forward_token(self.handle, tok, C.byref(out)), "engine_forward_token")
        return self._hidden(out)

    def forward_chunk(self, toks: Sequence[int]) -> torch.Tensor:
        ids = (C.c_uint32 * len(toks))(*toks)
        out = C.c_void_p()
        self.stream.wait_stream(torch.cuda.current_stream())
        check(lib().sph_engine_forward_chunk(self.handle, ids, len(toks), C.byref(out)), "engine_forward_chunk")
        return self._hidden(out)

    def use_graph(self, on: bool) -> None:
        check(lib().sph_engine_use_graph(self.handle, int(on)), "engine_use_graph")

    def reset(self) -> None:
        check(lib().sph_engine_reset(self.handle), "engine_reset")

    @property
    def position(self) -> int:
        return lib().sph_engine_position(self.handle)

    def cache(self, layer: int, which: str = "k") -> torch.Tensor:
        """Device view of a layer's K or V cache [n_kv_heads, max_seq, head_dim] (BF16 as raw uint16 bits)."""
        fn = lib().sph_engine_kcache if which == "k" else lib().sph_engine_vcache
        ptr = fn(self.handle, layer)
        torch.cuda.current_stream().wait_stream(self.stream)
        c = self.cfg
        t = torch.as_tensor(_DevArray(ptr, (c.n_kv_heads, c.max_seq, c.head_dim), _TYPESTR[c.kv_dtype]),
                            device="cuda")
        return t.view(torch.bfloat16) if c.kv_dtype == _lib.BF16 else t
