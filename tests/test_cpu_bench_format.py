"""CPU checks of bench.py's output format (no GPU): the final JSON line keeps every benchmark
configuration's row in compact form and stays well inside the 8 KB a log tail keeps; rows of
the full table carry what the compact form drops."""
import importlib.util
import json
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def _bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _row(op, dtype, cfg, latency=False):
    r = {"op": op, "shape": "8192x14336" if not latency else "512x896", "dtype": dtype, "cfg": cfg,
         "us": 112.34, "GB/s": 6272.3, "pct_peak": 78.4, "rows/s": 72919567.1, "alg_bytes": 704643072,
         "latency_bound": latency, "rotation_bytes": 1409286144, "sets": 2, "cpu_rows/s": 42.1, "cpu_sample": 64,
         "gpu_vs_cpu": 1731.9, "sclk_mhz": 2311.0, "torch_ref": "torch mul", "torch_ref_us": 118.7,
         "us_method": "rocprofv3 kernel trace of a child process, median of 200 launches per row"}
    if latency:
        r.update({"graph_us": 2.41, "call_us": 6.11, "kernel": "rms_rows_vec<float, float, float, 0, 2, 2, false>"})
    return r


def test_compact_rows_keep_identity_and_measurements():
    b = _bench()
    c = b.compact(_row("swiglu", "f16", 4))
    assert c["op"] == "swiglu" and c["cfg"] == 4 and c["us"] == 112.34 and c["pct_peak"] == 78.4
    assert c["torch_ref_us"] == 118.7 and "us_method" not in c and "alg_bytes" not in c


def test_final_line_fits_a_log_tail():
    """Twenty configuration rows (the count the default run prints) plus a headline line of the
    real field set (the host-tensor rate included) stay under 7 KB."""
    b = _bench()
    rows = ([_row("add_rms_norm", dt, 2) for dt in ("f16 (f32 w)", "bf16 (f32 w)")] +
            [_row(op, dt, 3) for op in ("rope_neox", "rope_interleaved") for dt in ("f32", "f16")] +
            [_row("swiglu", "f16", 4), _row("gelu_tanh", "f16", 4)] +
            [_row("embed_q4_k " + d, "q4_k->f32", 5) for d in ("uniform", "zipf1.1")] +
            [_row(f"{op} qwen T={t}", "f32", 1, latency=True) for t in (1, 512)
             for op in ("rms_norm", "add_rms_norm", "rope_neox", "swiglu", "embed_q8_0")])
    assert len(rows) == 20
    line = {"metric": b.METRIC, "value": 6113.8, "unit": "GB/s", "n_gpus": 1, "steps": 20, "warmup": 5,
            "ms_per_step": 0.1752, "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
            "data": "synthetic (seeded torch.randn ~N(0,1) inputs/residual, weight ~N(1,0.1); torch.Generator "
                    "seeds: x 10 and 11, residual 20 and 21 (two rotating sets), weight 3)",
            "config": {"workload": "fused residual-add + RMSNorm, Llama-3-8B width", "rows": 16384, "dim": 4096},
            "roofline": {"bound": "hbm", "achieved": 6113.8, "peak": 8000.0, "unit": "GB/s", "frac": 0.7642,
                         "traffic": 1073887092.0, "kernel": b.HEADLINE_KERNEL, "alg_bytes_per_launch": 1073758208,
                         "avg_launch_us": 175.23},
            "cpu_baseline": {"value": 11.9, "unit": "GB/s", "cores": 1, "kind": "port",
                             "sample": "oracle add_rms_norm on 2048x4096 f32 rows (1/8 of the workload), 889 reps in "
                                       "10 s, 1 thread of AMD EPYC 9575F 64-Core Processor (16 host cores visible)"},
            "plain_copy": {"kernel": "torch neg, 2 x 16384 x 4096 f32 (read + write)", "GB/s": 6120.2, "pct_peak": 76.5},
            "device_clock": {"sclk_mhz_during_headline": {"median": 825.0, "min": 711, "max": 893}, "samples": 14,
                             "sclk_levels": "0: 500Mhz 1: 1412Mhz * 2: 2400Mhz", "mclk": "0: 2000Mhz *",
                             "power_cap_w": 1400},
            "timing": {"region_ms": 3.505, "host_wall_ms": 3.747, "rotation_bytes": 1610612736,
                       "method": "one HIP event pair around the timed launches on their stream"},
            "ops": [b.compact(r) for r in rows],
            "ops_note": "x" * 300,
            "host_tensor": {"op": "add_rms_norm", "shape": "16384x4096 f32", "ms": 12.301, "GB/s": 87.3,
                            "first_call_ms": 32.55, "embed_one_id_ms": 0.0431, "decode_row_us": 16.7,
                            "how": "y" * 190},
            "children_left": 0}
    text = json.dumps(line)
    assert len(text) < 7000, len(text)
    assert all(r["cfg"] in (1, 2, 3, 4, 5) for r in line["ops"])
