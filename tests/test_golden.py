"""The committed fixture tests/golden/reference_vectors.npz (made by
tests/golden/make_golden.py from the reference tests' own generators):

  CPU: its inputs rebuild bit for bit from the generators (provenance), its
       dequant expectations are the reference tests' own, and today's oracle
       (and the libm it binds) still reproduces every frozen output bit for bit.
  GPU: the HIP kernels reproduce the frozen outputs (bit-exact ops) or stay
       within their stated tolerance of them.
"""
from pathlib import Path

import numpy as np
import pytest

import oracle
from golden.make_golden import build

FIX = Path(__file__).resolve().parent / "golden" / "reference_vectors.npz"


@pytest.fixture(scope="module")
def fx():
    with np.load(FIX, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_fixture_rebuilds_and_oracle_reproduces_it(fx):
    fresh = build()
    assert set(fresh) == set(fx)
    for k in fx:
        a, b = fresh[k], fx[k]
        assert a.shape == b.shape and a.dtype == b.dtype, k
        if a.dtype.kind == "f":
            nan = np.isnan(a) & np.isnan(b)
            assert np.array_equal(_bits(a)[~nan.reshape(-1)] if a.ndim == 1 else _bits(a)[~nan],
                                  _bits(b)[~nan.reshape(-1)] if b.ndim == 1 else _bits(b)[~nan]), k
        else:
            assert np.array_equal(a, b), k


def test_fixture_dequant_expectations_match_oracle(fx):
    assert np.array_equal(_bits(oracle.dequant(fx["q8_blocks"], oracle.Q8_0, fx["q8_deq"].size)), _bits(fx["q8_deq"]))
    assert np.array_equal(_bits(oracle.dequant(fx["q4k_blocks"], oracle.Q4_K, fx["q4k_deq"].size)), _bits(fx["q4k_deq"]))
    assert np.array_equal(_bits(oracle.dequant(fx["q6k_blocks"], oracle.Q6_K, fx["q6k_deq"].size)), _bits(fx["q6k_deq"]))


@pytest.mark.gpu
def test_gpu_reproduces_fixture(dev, fx):
    import torch
    import sapient_amd.ops as ops
    from helpers import max_rel, to_np
    from sapient_amd._lib import Q4_K, Q6_K, Q8_0

    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    # bit-exact ops
    assert np.array_equal(_bits(to_np(ops.add(t(fx["ew_a"]), t(fx["ew_b"])))), _bits(fx["add_out"]))
    assert np.array_equal(_bits(to_np(ops.gelu_tanh(t(fx["gelu_x"])))), _bits(fx["gelu_out"]))
    for key, dt, vocab, dim in (("q8", Q8_0, 100, 320), ("q4k", Q4_K, 50, 512), ("q6k", Q6_K, 40, 512)):
        ids = np.arange(vocab, dtype=np.uint32)[::-1].copy()
        out = ops.embed(t(fx[f"{key}_blocks"]), dt, vocab, dim, t(ids.view(np.int32)))
        assert np.array_equal(_bits(to_np(out)), _bits(fx[f"{key}_deq"].reshape(vocab, dim)[ids])), key
    # tolerance ops
    out = ops.rms_norm(t(fx["rms_x"]), t(fx["rms_w"]), 1e-5)
    assert max_rel(to_np(out), fx["rms_out"]) <= 1e-5
    assert max_rel(to_np(ops.swiglu(t(fx["ew_a"]), t(fx["ew_b"]))), fx["swiglu_out"], floor=1e-37) <= 1e-5
    for tag, rd in (("a", 32), ("b", 64)):
        for il in (False, True):
            x = t(fx[f"rope_{tag}_x"])
            ops.rope_(x, None, t(fx[f"rope_{tag}_pos"].astype(np.int32)), 1e4, rotary_dim=rd, interleaved=il)
            want = fx[f"rope_{tag}_il" if il else f"rope_{tag}_neox"]
            assert np.abs(to_np(x) - want).max() <= 1e-5 * np.abs(fx[f"rope_{tag}_x"]).max() * 1.5
