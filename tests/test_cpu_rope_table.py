"""CPU checks of sph_rope_table, the host function that evaluates RoPE angles for
the table-driven kernel (no device work, so these run without a GPU).

Reference: crates/sapient-backends/cpu/src/kernels/rope.rs:48-50 / :123-125 (the
angle and its sin_cos) and :140-153 (rope_cos_sin_cache, the table layout).

Pins: rotating unit pairs (x_i = 1, x_{i+half} = 0) with the oracle's RoPE
returns exactly (cos, sin) of each angle — 1·c − 0·s = c and 0·c + 1·s = s are
exact — so the table must equal the oracle's rotation of unit vectors bit for
bit; position 0 gives (1, 0) for every pair; a float64 evaluation of the same
angle agrees within f32 rounding; positions given explicitly and the implicit
0 .. n - 1 agree."""
import math

import numpy as np
import pytest


@pytest.fixture(scope="module")
def L():
    import sapient_amd
    if not sapient_amd.LIB_PATH.exists():
        from sapient_amd import build
        build.build()
    import torch  # noqa: F401  (load order: share torch's HIP runtime)
    from sapient_amd import _lib
    return _lib


def _table(positions, rd, base, scale=1.0, n=None):
    import sapient_amd.ops as ops
    return ops.rope_table(positions, rd, base, scale, n=n)


def _unit_rotation(orc, positions, rd, base, scale):
    """The oracle's RoPE of unit pairs: [S, rd] → (cos [S, half], sin [S, half])."""
    half = rd // 2
    x = np.zeros((1, 1, len(positions), rd), np.float32)
    x[..., :half] = 1.0
    out = orc.apply_rope_partial_scaled(x, positions, base, rd, scale)
    return out[0, 0, :, :half], out[0, 0, :, half:]


@pytest.mark.parametrize("rd,base,scale", [(128, 5e5, 1.0), (64, 1e6, 1.0), (32, 1e4, 1.0), (128, 1e6, 8.0),
                                           (6, 1e4, 1.0), (80, 1e4, 0.25)])
def test_table_equals_oracle_rotation_of_unit_pairs(L, orc, rd, base, scale):
    rng = np.random.default_rng(rd)
    positions = [0, 1, 2, 7, 4095, 8191, 131071] + [int(p) for p in rng.integers(0, 1 << 20, 64)]
    cs, sn = _table(positions, rd, base, scale)
    want_c, want_s = _unit_rotation(orc, positions, rd, base, scale)
    assert np.array_equal(cs.view(np.uint32), want_c.view(np.uint32))
    assert np.array_equal(sn.view(np.uint32), want_s.view(np.uint32))


def test_implicit_positions_are_the_reference_cache(L, orc):
    """positions None: rows 0 .. n - 1, rope_cos_sin_cache(n, head_dim, base) (rope.rs:140-153)."""
    n, hd, base = 300, 64, 1e6
    cs, sn = _table(None, hd, base, n=n)
    c2, s2 = _table(list(range(n)), hd, base)
    assert np.array_equal(cs.view(np.uint32), c2.view(np.uint32)) and np.array_equal(sn.view(np.uint32),
                                                                                      s2.view(np.uint32))
    assert (cs[0] == 1.0).all() and (sn[0] == 0.0).all()  # position 0: the identity rotation
    want_c, want_s = _unit_rotation(orc, list(range(n)), hd, base, 1.0)
    assert np.array_equal(cs, want_c) and np.array_equal(sn, want_s)


def test_table_near_float64_angles(L):
    """The f32 angle pos / base^(2i/d) and its sin / cos agree with a float64 evaluation to within the
    f32 rounding of the angle (a transposed exponent or a dropped scale would not)."""
    rd, base = 128, 5e5
    positions = list(range(0, 4096, 37))
    cs, sn = _table(positions, rd, base)
    for r, p in enumerate(positions):
        for i in range(0, rd // 2, 5):
            a = p / base ** (2 * i / rd)
            tol = 4 * abs(a) * 2.0 ** -23 + 1e-6
            assert abs(cs[r, i] - math.cos(a)) <= tol and abs(sn[r, i] - math.sin(a)) <= tol, (p, i)


def test_table_rejects_bad_arguments(L):
    import ctypes
    lib = L.lib()
    buf = (ctypes.c_float * 64)()
    neg = (ctypes.c_int64 * 2)(3, -1)
    assert lib.sph_rope_table(neg, 2, 8, 1e4, 1.0, buf, buf) == L.EINVAL          # negative position
    assert lib.sph_rope_table(None, 2, 7, 1e4, 1.0, buf, buf) == L.EINVAL         # odd rotary_dim
    assert lib.sph_rope_table(None, 2, 8, 1e4, 0.0, buf, buf) == L.EINVAL         # pos_scale 0
    assert lib.sph_rope_table(None, 2, 8, 1e4, float("nan"), buf, buf) == L.EINVAL
    assert lib.sph_rope_table(None, 2, 8, 1e4, 1.0, None, buf) == L.EINVAL
    assert lib.sph_rope_table(None, 0, 8, 1e4, 1.0, None, None) == L.OK           # nothing to fill
