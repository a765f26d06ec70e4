"""GPU test: the C ABI is stateless and reentrant, ordered per stream.

Four host threads, each with its own HIP stream and its own buffers, run the same
sequence of calls (fused add + RMSNorm, SwiGLU, half-precision GELU through the
per-device tables, RoPE, the Q8_0 gather, the KV-cache window update) many times
at once; every thread's final buffers must equal one serial run of the sequence
on the same inputs, bit for bit, and the serial run is checked against the
oracle. (ctypes releases the interpreter lock around each call, so the threads'
calls do overlap in the library.)
"""
import threading

import numpy as np
import pytest
import torch

from helpers import assert_bits_equal, max_rel, to_np, widen

import sapient_amd.ops as ops
from sapient_amd._lib import Q8_0

pytestmark = pytest.mark.gpu
THREADS, ROUNDS = 4, 25
ROWS, DIM, INTER, H, S, D = 16, 896, 4864, 14, 8, 64
VOCAB = 64


def _inputs(dev, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    r = lambda *shape, dt=torch.float32: torch.randn(*shape, generator=g, device=dev).to(dt)
    rng = np.random.default_rng(seed)
    nb = VOCAB * DIM // 32
    blocks = rng.integers(0, 256, (nb, 34), dtype=np.uint8)
    blocks[:, 0:2] = np.frombuffer(rng.uniform(-0.05, 0.05, nb).astype(np.float16).tobytes(), np.uint8).reshape(nb, 2)
    return dict(x=r(ROWS, DIM), res=r(ROWS, DIM), w=r(DIM) * 0.1 + 1, gate=r(ROWS, INTER), up=r(ROWS, INTER),
                hx=r(ROWS, INTER, dt=torch.float16), q=r(1, H, S, D), k=r(1, 2, S, D),
                pos=torch.arange(100, 100 + S, dtype=torch.int32, device=dev),
                table=torch.from_numpy(blocks.reshape(-1)).to(dev),
                ids=torch.from_numpy(rng.integers(0, VOCAB, 40).astype(np.int32)).to(dev),
                src=r(2, 1, D), cache=r(2, 32, D, dt=torch.float16))


def _sequence(t, rounds):
    """The calls, on the current stream; returns the buffers they produced."""
    res = t["res"].clone()
    q, k, cache = t["q"].clone(), t["k"].clone(), t["cache"].clone()
    nxt = torch.empty_like(cache)
    for _ in range(rounds):
        y, _ = ops.add_rms_norm(t["x"], res, t["w"], 1e-6)
        sg = ops.swiglu(t["gate"], t["up"])
        hg = ops.gelu_tanh(t["hx"])
        ops.rope_(q, k, t["pos"], 1e6)
        e = ops.embed(t["table"], Q8_0, VOCAB, DIM, t["ids"])
        ops.kv_cache_update_into(t["src"], cache, nxt, 32)
        cache, nxt = nxt, cache
    return dict(y=y, res=res, sg=sg, hg=hg, q=q, k=k, e=e, cache=cache)


def test_threads_on_their_own_streams_equal_a_serial_run(dev, orc):
    inputs = [_inputs(dev, 11 + i) for i in range(THREADS)]
    torch.cuda.synchronize()
    serial = []
    for t in inputs:
        serial.append({n: v.clone() for n, v in _sequence(t, ROUNDS).items()})
    torch.cuda.synchronize()
    # the serial run against the oracle (first thread's inputs; the residual after ROUNDS adds of x)
    t0, s0 = inputs[0], serial[0]
    r32 = to_np(t0["res"]).copy()
    for _ in range(ROUNDS):
        y32, r32 = orc.add_rms_norm(to_np(t0["x"]), r32, to_np(t0["w"]), 1e-6)
    assert_bits_equal(to_np(s0["res"]), r32, "serial residual")
    assert max_rel(to_np(s0["y"]), y32) <= 1e-5
    assert_bits_equal(to_np(s0["sg"]), orc.swiglu(to_np(t0["gate"]), to_np(t0["up"])), "serial swiglu")
    assert np.array_equal(to_np(s0["hg"]), orc.f32_to_f16_bits(orc.gelu(widen(t0["hx"], orc))))
    print(f"case concurrency: {THREADS} threads x {ROUNDS} rounds", flush=True)
    results, errors = [None] * THREADS, []

    def worker(i):
        try:
            s = torch.cuda.Stream()
            with torch.cuda.stream(s):
                out = _sequence(inputs[i], ROUNDS)
            s.synchronize()
            results[i] = out
        except Exception as exc:  # reported below, on the main thread
            errors.append((i, repr(exc)))

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(THREADS)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=120)
    assert not any(th.is_alive() for th in threads), "a worker did not finish"
    assert not errors, errors
    bits = lambda t: to_np(t).view(np.uint32) if t.dtype == torch.float32 else to_np(t)
    for i in range(THREADS):
        for name, want in serial[i].items():
            assert np.array_equal(bits(results[i][name]), bits(want)), f"thread {i} {name}"
