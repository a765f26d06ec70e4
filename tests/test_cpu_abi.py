"""CPU-only checks of the boundary: the built library loads, exports exactly the
symbols the C headers under include/ declare, and its ctypes binding covers
them. No kernel is launched (there is no GPU here)."""
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADERS = sorted((ROOT / "include").glob("*.h"))


def declared_symbols() -> set[str]:
    text = "\n".join(h.read_text() for h in HEADERS)
    return set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(sph_\w+)\s*\(", text, flags=re.M))


@pytest.fixture(scope="module")
def built_lib():
    import sapient_amd
    if not sapient_amd.LIB_PATH.exists():
        from sapient_amd import build
        build.build()
    return sapient_amd.LIB_PATH


def test_header_declares_the_op_set():
    syms = declared_symbols()
    for s in ("sph_rms_norm", "sph_add_rms_norm", "sph_add", "sph_mul", "sph_silu", "sph_swiglu",
              "sph_gelu_tanh", "sph_rope", "sph_embed", "sph_status_string", "sph_abi_version", "sph_init"):
        assert s in syms, s


def test_library_exports_every_declared_symbol(built_lib):
    out = subprocess.run(["nm", "-D", "--defined-only", str(built_lib)], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r"\sT\s(sph_\w+)$", out, flags=re.M))
    assert declared_symbols() == exported


def test_library_loads_and_binding_covers_header(built_lib):
    import torch  # noqa: F401  (load order: share torch's HIP runtime)
    from sapient_amd import _lib
    L = _lib.lib()
    assert set(_lib.SIGNATURES) == declared_symbols()
    assert L.sph_abi_version() == 1
    assert L.sph_status_string(_lib.ERANGE).startswith(b"index out of range")
    assert L.sph_status_string(12345) == b"unknown status"


def test_argument_validation_needs_no_device(built_lib):
    """Rejections happen on the host before any HIP call."""
    from sapient_amd import _lib
    L = _lib.lib()
    E = _lib.EINVAL
    assert L.sph_rms_norm(None, 0, None, 0, None, 0, -1, 8, 1e-5, None) == E
    assert L.sph_rms_norm(None, 0, None, 0, None, 0, 0, 8, 1e-5, None) == _lib.OK  # empty
    assert L.sph_add(None, 3, None, 3, None, 0, None) == E
    assert L.sph_add(1, 3, 2, 2, 3, 0, None) == E                                  # lengths 3 vs 2
    assert L.sph_swiglu(None, None, None, 0, -1, None) == E
    assert L.sph_gelu_tanh(None, None, 7, 0, None) == E
    assert L.sph_rope(None, 1, None, 0, 0, 0, None, 1, 1, 7, 7, 1e4, 1.0, None) == E    # odd head_dim
    assert L.sph_rope(None, 1, None, 0, 0, 0, None, 1, 1, 8, 10, 1e4, 1.0, None) == E   # rotary > head
    assert L.sph_rope(None, 1, None, 0, 0, 5, None, 1, 1, 8, 8, 1e4, 1.0, None) == E    # layout
    assert L.sph_embed(None, 8, 10, 48, None, 1, None, None, None) == E                 # 48 % 32
    assert L.sph_embed(None, 12, 10, 512, None, 0, None, None, None) == _lib.OK         # no ids
    assert L.sph_embed(None, 3, 10, 512, None, 1, None, None, None) == E                # Q4_1: not a table type
    assert L.sph_embed(None, 2, 10, 48, None, 1, None, None, None) == E                 # Q4_0: 48 % 32
    assert L.sph_embed(None, 13, 10, 512, None, 0, None, None, None) == _lib.OK         # Q5_K, no ids
    tok = lambda q, qo, seq: L.sph_rope_kv_append_tokens(q, qo, 2, 64, 64, 1, 0, 0, 64, seq, 64, 1e4, 1.0, 64, 64, 0,
                                                         16, None, None, None, 0, None, None)
    assert tok(4096, 4096, 3) == E                                                     # q_out overlaps q
    assert tok(4096, None, 3) == E                                                     # no q_out
    assert tok(4096, 4096, 0) == _lib.OK                                               # empty chunk
