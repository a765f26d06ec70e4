"""Writes tests/golden/reference_vectors.npz: the input vectors of the reference's
own tests, rebuilt with their generators (tests/refvec.py), with

  - the expected values those tests compute in-test (dequant restatements), and
  - the oracle's outputs on the same inputs, frozen when this file was run
    (glibc 2.35 libm: expf, tanhf, powf, sinf, cosf).

The fixture lets a later run detect a drift of the oracle or of the libm it
binds. Regenerate with `python tests/golden/make_golden.py` (CPU only).
"""
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))
sys.path.insert(0, str(HERE.parent))

import oracle  # noqa: E402
from refvec import (WgpuLcg, f16_bits, gather_test_values, quantize_q8_0_blocks, random_q4_k_blocks,  # noqa: E402
                    random_q6_k_blocks)


def build() -> dict:
    v = {}
    # resident.rs:28-59 (rms_norm 5 x 1536, seed 0x12345678)
    nxt = WgpuLcg(0x12345678)
    v["rms_x"] = nxt.take(5 * 1536).reshape(5, 1536)
    v["rms_w"] = np.float32(0.5) + np.abs(nxt.take(1536))
    v["rms_out"] = oracle.rms_norm(v["rms_x"], v["rms_w"], 1e-5)
    # resident.rs:103-124 (add / swiglu n = 4096)
    nxt = WgpuLcg()
    v["ew_a"], v["ew_b"] = nxt.take(4096), nxt.take(4096)
    v["add_out"] = oracle.add(v["ew_a"], v["ew_b"])
    v["swiglu_out"] = oracle.swiglu(v["ew_a"], v["ew_b"])
    v["silu_out"] = oracle.silu(v["ew_a"])
    # resident.rs:909-930 data (lcg * 4, n = 4133) for GELU (tanh) and erf-GELU
    v["gelu_x"] = WgpuLcg().take(4096 + 37) * np.float32(4.0)
    v["gelu_out"] = oracle.gelu(v["gelu_x"])
    v["gelu_erf_out"] = oracle.gelu_erf(v["gelu_x"])
    # resident.rs:152-187 (rope (4,7,80,32) and (3,5,64,64), positions s + 11, base 1e4)
    for tag, (H, S, D, rd) in (("a", (4, 7, 80, 32)), ("b", (3, 5, 64, 64))):
        x = WgpuLcg().take(H * S * D).reshape(1, H, S, D)
        pos = np.arange(S) + 11
        v[f"rope_{tag}_x"], v[f"rope_{tag}_pos"] = x, pos
        v[f"rope_{tag}_neox"] = oracle.apply_rope_partial_scaled(x, pos, 1e4, rd)
        v[f"rope_{tag}_il"] = oracle.apply_rope_partial_scaled(x, pos, 1e4, rd, 1.0, interleaved=True)
    # resident.rs:565-592 (embed q8_0 100 x 320), :678-705 (embed q4_k 50 x 512), q6_k generator
    table = WgpuLcg().take(100 * 320)
    v["q8_blocks"], v["q8_deq"] = quantize_q8_0_blocks(table)
    v["q4k_blocks"], v["q4k_deq"] = random_q4_k_blocks(50 * 512 // 256, WgpuLcg())
    v["q6k_blocks"], v["q6k_deq"] = random_q6_k_blocks(40 * 512 // 256, WgpuLcg())
    # common.rs:678-718 (gather vs full dequant, vocab 17 x 256, seed 0xABCD)
    data = gather_test_values()
    v["gather_data"], v["gather_f16"] = data, f16_bits(data)
    v["gather_q8"] = oracle.quantize_q8_0(data)
    v["gather_ids"] = np.array([0, 7, 16, 3], np.uint32)
    return v


if __name__ == "__main__":
    out = HERE / "reference_vectors.npz"
    np.savez_compressed(out, **build())
    print(f"wrote {out} ({out.stat().st_size} bytes)")
