#!/usr/bin/env python3
"""Benchmark of the fused per-layer op set on one MI355X.

Headline step: one fused residual-add + RMSNorm launch over 16384 x 4096 f32
(Llama-3-8B width, eps 1e-5) — x and residual in, normed rows and the updated
residual out, every input resident in HBM before timing starts. The last
JSON line reports that kernel's achieved HBM bandwidth (algorithmic bytes x
launches / the time of the K back-to-back launches between one HIP event pair
on their stream; one untimed launch goes ahead of the start event so the
region holds GPU work only) against MI355X's 8 TB/s, the single-thread CPU
oracle on a bounded sample of the same workload, and (``ops``, compact) the
same measurement for the rows of the five benchmark configurations. The line
before it (``ops_full``) holds every row in full, the configuration rows and
the others (other dtypes and table formats, LayerNorm, erf-GELU, the layout
helpers, the decode engine).

Every throughput row rotates buffer sets totalling at least 512 MiB
(``rotation_bytes``), so the 256 MB Infinity Cache cannot serve a repeat; the
gather rows rotate whole tables and id sets. Each starts after half a second
of idle and at least 25 ms of warm-up launches. Rows whose launches take under
25 us are timed as back-to-back launches replayed from a HIP graph (Python
issues a launch in ~10 us, which would otherwise be what the events measure).
The latency-bound Qwen2.5-0.5B rows report kernel durations from a rocprofv3
kernel trace of a child process (``us``), beside the per-launch time of a
replayed HIP graph of back-to-back launches (``graph_us``) and one call's
latency from the host (``call_us``).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-ops] [--cpu-seconds S]
"""
from __future__ import annotations

import argparse
import csv
import json
import os
import re
import shutil
import signal
import subprocess
import sys
import tempfile
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "fused-op HBM GB/s & % of 8 TB/s peak (RMSNorm/RoPE/SwiGLU/embed)"
PEAK_GBS = 8000.0
PROFILES = ROOT / "profiles"
# The headline's kernel instantiation (fused add + RMSNorm, f32, 16 waves per row, one
# 16-byte vector per lane, row-looping blocks), as rocprofv3 names it.
HEADLINE_KERNEL = "rms_rows_vec<float, float, float, 1, 16, 1, true>"
# Every throughput row rotates at least this many bytes of distinct buffers (twice the
# 256 MB Infinity Cache), so no launch can be served from the previous launches' lines.
ROTATION_MIN = 1 << 29
# Launches per latency-bound row in the kernel-trace child (the first C1_SKIP are warm-up).
C1_LAUNCHES, C1_SKIP = 220, 20
# Throughput rows whose event-timed launches take less than this (ms) are re-timed from a HIP graph.
SHORT_MS = 0.025
# Idle seconds before each throughput row (see op_table).
SETTLE_S = 0.5


def parse():
    p = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=100, help="untimed headline launches before the timed ones "
                   "(100: ~17 ms, enough for the GPU to reach steady clocks)")
    p.add_argument("--no-ops", action="store_true", help="skip the per-op table")
    p.add_argument("--only", default=None, help="comma list of op names for the per-op table")
    p.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU-baseline time budget")
    p.add_argument("--op-cpu-seconds", type=float, default=0.3, help="CPU time budget per op-table row")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--no-host-tensor", action="store_true",
                   help="skip the C++ trait mirror's host-tensor rate (a child process)")
    p.add_argument("--no-kernel-trace", action="store_true",
                   help="latency-bound rows: skip the rocprofv3 child (us = graph replay per launch)")
    p.add_argument("--profile-run", action="store_true",
                   help="launch only the headline kernel (warmup + steps) and the calibration copies: for "
                        "rocprofv3; with --only, the named op-table rows instead of the headline")
    p.add_argument("--latency-child", action="store_true", help=argparse.SUPPRESS)
    return p.parse_args()


# ───────────────────────────── timing helpers ─────────────────────────────
def time_launches(torch, fn, sets, warmup: int, steps: int):
    """Run fn(set) over rotating buffer sets; return per-launch ms (HIP events on
    the current stream, the stream every op is enqueued on)."""
    stream = torch.cuda.current_stream()
    for i in range(warmup):
        fn(sets[i % len(sets)])
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    t0 = time.perf_counter()
    for i in range(steps):
        s, e = evs[i]
        s.record(stream)
        fn(sets[i % len(sets)])
        e.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per = [s.elapsed_time(e) for s, e in evs]
    return per, wall


def time_region(torch, fn, sets, warmup: int, steps: int):
    """Run fn(set) over rotating buffer sets: `warmup` untimed, then exactly `steps` timed launches
    between one HIP event pair on the current stream (the stream every op is enqueued on), with
    synchronizations before and after. One more untimed launch goes ahead of the start event: the GPU
    runs it while the host queues the timed ones, so the region holds the `steps` launches back to
    back and not the host's latency to queue the first of them. Returns (ms for the whole region,
    host wall seconds)."""
    stream = torch.cuda.current_stream()
    for i in range(warmup):
        fn(sets[i % len(sets)])
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    fn(sets[warmup % len(sets)])  # the lead launch (untimed)
    start.record(stream)
    for i in range(steps):
        fn(sets[(warmup + 1 + i) % len(sets)])
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end), time.perf_counter() - t0


def median(xs):
    return float(np.median(np.asarray(xs)))


def warm(torch, fn, sets, min_launches: int = 3, min_ms: float = 25.0):
    """Untimed launches until at least `min_launches` ran and `min_ms` of GPU time passed, so that
    the row is timed at steady clocks (the GPU idles while the CPU columns are measured)."""
    t0 = time.perf_counter()
    i = 0
    while True:
        fn(sets[i % len(sets)])
        i += 1
        if i >= min_launches and i % len(sets) == 0:
            torch.cuda.synchronize()
            if (time.perf_counter() - t0) * 1e3 >= min_ms:
                return


def time_regions(torch, fn, sets, regions: int = 5, steps: int = 20):
    """Steady-state per-launch ms: after `warm`, `regions` regions of `steps` back-to-back launches,
    each between one HIP event pair; the median region / steps."""
    warm(torch, fn, sets)
    steps = max(steps, len(sets))  # every region walks the whole rotation at least once
    return median([time_region(torch, fn, sets, 0, steps)[0] for _ in range(regions)]) / steps


def time_graph(torch, fn, sets, launches: int = 200, replays: int = 5):
    """Per-launch ms of `launches` back-to-back launches captured into one HIP graph and replayed
    (kernel time plus the dispatch gap between dependent kernels); the median of `replays`."""
    for i in range(4):
        fn(sets[i % len(sets)])
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(launches):
            fn(sets[i % len(sets)])
    g.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    per = []
    for _ in range(replays):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        g.replay()
        end.record(stream)
        torch.cuda.synchronize()
        per.append(start.elapsed_time(end) / launches)
    del g
    return median(per)


def cpu_time(fn, budget_s: float, min_reps: int = 1):
    """Repeat fn until the budget is spent; return (seconds per call, reps)."""
    fn()  # first touch of the output pages
    reps, t0 = 0, time.perf_counter()
    while True:
        fn()
        reps += 1
        el = time.perf_counter() - t0
        if reps >= min_reps and el >= budget_s:
            return el / reps, reps


def committed_traffic(kernel_tag: str):
    """HBM bytes per launch of the headline kernel from the committed rocprofv3
    --pmc summary (FETCH_SIZE + WRITE_SIZE, calibrated), or None."""
    f = PROFILES / f"{kernel_tag}_pmc.md"
    if not f.exists():
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", f.read_text())
    return float(m.group(1)) if m else None


# ───────────────────────────── buffer sets ─────────────────────────────
def set_bytes(torch, s) -> int:
    """Bytes of the distinct tensors one buffer set holds."""
    seen = {}

    def walk(o):
        if isinstance(o, torch.Tensor):
            seen[o.data_ptr()] = o.numel() * o.element_size()
        elif isinstance(o, (list, tuple)):
            for x in o:
                walk(x)
    walk(s)
    return sum(seen.values())


def rotation(torch, make_set, min_bytes: int = ROTATION_MIN, min_sets: int = 2):
    """Buffer sets make_set(0), make_set(1), ... until they hold at least `min_bytes` (and at least
    `min_sets` sets). Returns (sets, bytes rotated)."""
    sets = [make_set(0)]
    per = set_bytes(torch, sets[0])
    n = max(min_sets, -(-min_bytes // max(per, 1)))
    sets += [make_set(i) for i in range(1, n)]
    return sets, sum(set_bytes(torch, s) for s in sets)


# ───────────────────────────── workloads ─────────────────────────────
def gen(torch, shape, seed, dev, dtype, std=1.0, mean=0.0):
    g = torch.Generator(device=dev).manual_seed(seed)
    return (torch.randn(shape, generator=g, device=dev) * std + mean).to(dtype)


def headline(torch, ops, dev, args, clocks=None):
    rows, dim = 16384, 4096
    f32 = torch.float32
    w = gen(torch, (dim,), 3, dev, f32, 0.1, 1.0)
    # two buffer sets (2 x 805 MB) so no launch can be served by the 256 MB Infinity Cache
    sets = [(gen(torch, (rows, dim), 10 + i, dev, f32), gen(torch, (rows, dim), 20 + i, dev, f32),
             torch.empty(rows, dim, device=dev)) for i in range(2)]

    def fn(s):
        ops.add_rms_norm(s[0], s[1], w, 1e-5, out=s[2])

    if clocks is not None:
        with clocks:
            region_ms, wall = time_region(torch, fn, sets, args.warmup, args.steps)
    else:
        region_ms, wall = time_region(torch, fn, sets, args.warmup, args.steps)
    alg_bytes = 4 * rows * dim * 4 + dim * 4  # read x, residual, weight; write y, residual
    return rows, dim, alg_bytes, region_ms, wall, sum(set_bytes(torch, s) for s in sets)


def engine_rows(torch, dev, table, vocab):
    import sapient_amd._lib as L
    from sapient_amd.engine import Engine
    f32 = torch.float32
    H, layers_n = 896, 24
    cfg = L.EngineConfig(H, 14, 2, 64, 4864, layers_n, 4096, 512, 1e-6, 1e6, L.ROPE_NEOX, L.F16, L.F32)
    layers = [dict(input_ln=gen(torch, (H,), 200 + l, dev, f32, 0.1, 1.0), post_ln=gen(torch, (H,), 300 + l, dev, f32, 0.1, 1.0),
                   bq=gen(torch, (896,), 400 + l, dev, f32, 0.1), bk=gen(torch, (128,), 500 + l, dev, f32, 0.1),
                   bv=gen(torch, (128,), 600 + l, dev, f32, 0.1), bo=None) for l in range(layers_n)]
    eng = Engine(cfg, table, L.Q8_0, vocab, layers, gen(torch, (H,), 700, dev, f32, 0.1, 1.0))
    rows = []
    for graph in (False, True):
        eng.reset()
        eng.use_graph(graph)
        for t in range(8):
            eng.forward_token(t)
        torch.cuda.synchronize()
        n = 256
        t0 = time.perf_counter()
        for t in range(n):
            eng.forward_token((t * 7919) % vocab)
        torch.cuda.synchronize()
        us = (time.perf_counter() - t0) / n * 1e6
        rows.append({"op": "engine decode token" + (" (graph)" if graph else " (eager)"),
                     "shape": "qwen2.5-0.5b 24 layers, op-set part", "dtype": "f32 act, f16 kv",
                     "us": round(us, 2), "tokens/s": round(1e6 / us, 1), "latency_bound": True,
                     "kernels_per_token": 1 + layers_n * 4 + 1})
    # A 4096-token prompt as eight 512-token chunks (positions 0 .. 4095), per chunk; the first pass
    # (untimed) fills the RoPE angle table.
    toks = [(t * 104729) % vocab for t in range(512)]
    eng.use_graph(False)
    reps = 4
    for r in range(reps + 1):
        if r == 1:
            torch.cuda.synchronize()
            t0 = time.perf_counter()
        eng.reset()
        for _ in range(8):
            eng.forward_chunk(toks)
    torch.cuda.synchronize()
    us = (time.perf_counter() - t0) / (reps * 8) * 1e6
    rows.append({"op": "engine prefill chunk", "shape": "qwen2.5-0.5b 24 layers, 8 x 512 tokens, op-set part",
                 "dtype": "f32 act, f16 kv", "us": round(us, 2), "tokens/s": round(512e6 / us, 1),
                 "latency_bound": True, "kernels_per_chunk": 1 + layers_n * 5 + 1})
    eng.close()
    return rows


class Row:
    """One op-table row: name, shape, dtype label, algorithmic bytes per launch, units per launch
    (rows / tokens / ids), make_set(i) -> the i-th buffer set, fn(set) -> one launch, and cpu() ->
    (oracle call, units it covers) for the CPU column."""

    def __init__(self, name, shape, dtype, alg_bytes, units, unit_name, make_set, fn, cpu=None, latency=False,
                 cfg=None, ref=None):
        self.name, self.shape, self.dtype, self.alg_bytes = name, shape, dtype, alg_bytes
        self.units, self.unit_name, self.make_set, self.fn, self.cpu = units, unit_name, make_set, fn, cpu
        self.latency = latency
        self.cfg = cfg  # the benchmark configuration (1-5) this row measures, or None for an extra row
        # (label, fn(set)): a torch kernel with the same memory traffic on the same buffers (a copy-like
        # reference: the same machine and buffer placement, a kernel this library did not write), or None
        self.ref = ref


def q_table(torch, dev, g, vocab, hidden, block, nbytes, d_off, nd, dmin=0.0005, dmax=0.02, signed_q=False):
    """A raw GGUF table [vocab, hidden] of `block`-element blocks of `nbytes` bytes: random quant
    bytes (int8 in [-127, 127] when signed_q) with `nd` f16 scales ~U(dmin, dmax) at byte d_off."""
    nb = vocab * hidden // block
    if signed_q:
        t = torch.randint(-127, 128, (nb, nbytes), generator=g, device=dev, dtype=torch.int32).to(torch.int8)
        t = t.view(torch.uint8)
    else:
        t = torch.randint(0, 256, (nb, nbytes), generator=g, device=dev, dtype=torch.int32).to(torch.uint8)
    dd = (torch.rand((nb, nd), generator=g, device=dev) * (dmax - dmin) + dmin).to(torch.float16)
    t[:, d_off:d_off + 2 * nd] = dd.view(torch.uint8).view(nb, 2 * nd)
    return t.reshape(-1)


def latency_rows(torch, ops, dev, orc, nrm, cpu_gather):
    """The Qwen2.5-0.5B (config 1) layer ops at T = 1 and T = 512: latency-bound, reported only."""
    import sapient_amd._lib as L
    f32, f16 = torch.float32, torch.float16
    H = 896
    rows = []
    for T1 in (1, 512):
        w = gen(torch, (H,), 3, dev, f32, 0.1, 1.0)
        rows.append(Row(f"rms_norm qwen T={T1}", f"{T1}x{H}", "f32", T1 * H * 8 + H * 4, T1, "rows",
                        lambda i, T1=T1: (gen(torch, (T1, H), 100 + i, dev, f32), torch.empty(T1, H, device=dev)),
                        lambda s, w=w: ops.rms_norm(s[0], w, 1e-6, out=s[1]),
                        lambda T1=T1: (lambda x=nrm(T1, H), w=nrm(H, scale=0.1, mean=1.0):
                                       orc.rms_norm(x, w, 1e-6), T1), latency=True, cfg=1))
        # The residual add fused into the next RMSNorm (llama.rs:508 -> :515): x and the residual read,
        # the normed rows and the updated residual written.
        rows.append(Row(f"add_rms_norm qwen T={T1}", f"{T1}x{H}", "f32", T1 * H * 16 + H * 4, T1, "rows",
                        lambda i, T1=T1: (gen(torch, (T1, H), 150 + i, dev, f32), gen(torch, (T1, H), 160 + i, dev, f32),
                                          torch.empty(T1, H, device=dev)),
                        lambda s, w=w: ops.add_rms_norm(s[0], s[1], w, 1e-6, out=s[2]),
                        lambda T1=T1: (lambda x=nrm(T1, H), r=nrm(T1, H), w=nrm(H, scale=0.1, mean=1.0):
                                       orc.add_rms_norm(x, r, w, 1e-6), T1), latency=True, cfg=1))
        # RoPE as the trait path's apply_rope_positions runs it: cos / sin from the backend's angle table
        # (positions 0 .. 63 at least, resident on the device, as rope_cos_sin_cache lays it out) at
        # device positions; the device sin/cos route beside it as an extra row.
        pos = torch.arange(T1, dtype=torch.int32, device=dev)
        cs, sn = (torch.from_numpy(t).to(dev) for t in ops.rope_table(None, 64, 1e6, n=max(64, T1)))
        qk = (lambda i, T1=T1: (gen(torch, (1, 14, T1, 64), 110 + i, dev, f32),
                                gen(torch, (1, 2, T1, 64), 120 + i, dev, f32)))
        rope_cpu = (lambda T1=T1: (lambda q=nrm(1, 16, T1, 64), p=np.arange(T1): orc.apply_rope(q, p, 1e6), T1))
        rows.append(Row(f"rope_neox qwen T={T1}", f"q14+k2 x {T1} x 64", "f32", 2 * 16 * T1 * 64 * 4 + T1 * (4 + 32 * 8),
                        T1, "tokens", qk, lambda s, cs=cs, sn=sn, pos=pos: ops.rope_cached_(s[0], s[1], cs, sn, pos),
                        rope_cpu, latency=True, cfg=1))
        rows.append(Row(f"rope_neox qwen T={T1} device-angles", f"q14+k2 x {T1} x 64", "f32", 2 * 16 * T1 * 64 * 4 + 4 * T1,
                        T1, "tokens", qk, lambda s, pos=pos: ops.rope_(s[0], s[1], pos, 1e6), rope_cpu, latency=True))
        rows.append(Row(f"swiglu qwen T={T1}", f"{T1}x4864", "f32", 3 * T1 * 4864 * 4, T1, "rows",
                        lambda i, T1=T1: (gen(torch, (T1, 4864), 130 + i, dev, f32),
                                          gen(torch, (T1, 4864), 140 + i, dev, f32), torch.empty(T1, 4864, device=dev)),
                        lambda s: ops.swiglu(s[0], s[1], out=s[2]),
                        lambda T1=T1: (lambda g=nrm(T1, 4864), u=nrm(T1, 4864): orc.swiglu(g, u), T1), latency=True,
                        cfg=1))
    vocab_q, hid_q = 151936, 896
    g = torch.Generator(device=dev).manual_seed(11)
    tq = q_table(torch, dev, g, vocab_q, hid_q, 32, 34, 0, 1, 0.001, 0.05, signed_q=True)
    rng = np.random.default_rng(12)
    for T1 in (1, 512):
        ids = [torch.from_numpy(rng.integers(0, vocab_q, T1).astype(np.int32)).to(dev) for _ in range(2)]
        rows.append(Row(f"embed_q8_0 qwen T={T1}", f"{vocab_q}x{hid_q} -> {T1} ids", "q8_0->f32",
                        T1 * (952 + 4 + hid_q * 4), T1, "rows",
                        lambda i, T1=T1, ids=ids: (ids[i % 2], torch.empty(T1, hid_q, device=dev)),
                        lambda s: ops.embed(tq, L.Q8_0, vocab_q, hid_q, s[0], out=s[1]),
                        lambda T1=T1: cpu_gather(L.Q8_0, 32, 34, 0, 1, hid_q, T1), latency=True, cfg=1))
    return rows, tq, vocab_q


def latency_kernel_times(rows_names):
    """Kernel durations of the latency-bound rows: this script re-run as a child under
    `rocprofv3 --kernel-trace` (each row's kernel launched C1_LAUNCHES times in order, one library
    kernel per launch); returns ({row name: median µs over the last C1_LAUNCHES - C1_SKIP}, note),
    or (None, reason) when the profiler is unavailable or its trace does not match the plan."""
    prof = shutil.which("rocprofv3")
    if prof is None:
        return None, "rocprofv3 not found"
    with tempfile.TemporaryDirectory(prefix="sph_c1_") as tmp:
        env = dict(os.environ, TMPDIR=tmp)
        cmd = [prof, "--kernel-trace", "--output-format", "csv", "-d", tmp, "-o", "c1", "--",
               sys.executable, str(ROOT / "bench.py"), "--latency-child"]
        # Its own process group, so a time-out ends the profiled program too, not only rocprofv3.
        child = subprocess.Popen(cmd, cwd=tmp, env=env, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True,
                                 start_new_session=True)
        try:
            out, _ = child.communicate(timeout=300)
        except subprocess.TimeoutExpired:
            os.killpg(child.pid, signal.SIGKILL)
            child.communicate()
            return None, "kernel-trace child timed out"
        plan = None
        for line in out.splitlines():
            if line.startswith('{"latency_child"'):
                plan = json.loads(line)
        traces = list(Path(tmp).rglob("c1_kernel_trace.csv"))
        if plan is None or not traces:
            return None, f"kernel-trace child failed (rc {child.returncode})"
        with open(traces[0], newline="") as f:
            recs = [r for r in csv.DictReader(f) if "sph::" in r["Kernel_Name"]]
        recs.sort(key=lambda r: int(r["Dispatch_Id"]))
        n = plan["launches"]
        if len(recs) != n * len(plan["rows"]) or plan["rows"] != rows_names:
            return None, f"kernel trace holds {len(recs)} library dispatches, expected {n * len(plan['rows'])}"
        out = {}
        for k, name in enumerate(plan["rows"]):
            durs = [(int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3 for r in recs[k * n:(k + 1) * n]]
            names = {r["Kernel_Name"] for r in recs[k * n:(k + 1) * n]}
            if len(names) != 1:
                return None, f"row {name}: more than one kernel per launch"
            kernel = names.pop().replace("sph::(anonymous namespace)::", "")
            out[name] = (median(durs[C1_SKIP:]), re.sub(r"^void |\(.*$", "", kernel))
        return out, f"rocprofv3 kernel trace of a child process, median of {n - C1_SKIP} launches per row"


def latency_child():
    """Child of latency_kernel_times: launch each latency-bound row's op C1_LAUNCHES times, in order."""
    import torch

    import sapient_amd.ops as ops
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    rows, _, _ = latency_rows(torch, ops, dev, None, None, None)
    for r in rows:
        sets = [r.make_set(i) for i in range(2)]
        torch.cuda.synchronize()
        for i in range(C1_LAUNCHES):
            r.fn(sets[i % 2])
        torch.cuda.synchronize()
    print(json.dumps({"latency_child": True, "launches": C1_LAUNCHES, "rows": [r.name for r in rows]}), flush=True)


def op_table(torch, ops, dev, only=None, cpu_budget=0.0, profile_launches=0, kernel_trace=True, clocks=None):
    """Per-op GB/s at each configuration shape (after >= 25 ms of warm-up launches, the median of 5
    regions of back-to-back launches between one event pair, over buffer sets rotating >= 512 MiB;
    latency-bound rows: kernel durations from a rocprofv3 trace, graph replay and one call's latency),
    and beside it the oracle — the reference's algorithm restated in C, one thread — on a sample of the
    same shape's rows (or tokens, ids), `cpu_budget` seconds each, reported in the same units.
    profile_launches > 0: only launch each selected row that many times (for rocprofv3), time nothing."""
    import sapient_amd._lib as L
    f32, f16, bf16 = torch.float32, torch.float16, torch.bfloat16
    res = []
    orc = None
    if cpu_budget > 0:
        import oracle as orc
    crng = np.random.default_rng(1)

    def nrm(*shape, scale=1.0, mean=0.0):
        return crng.standard_normal(shape, dtype=np.float32) * np.float32(scale) + np.float32(mean)

    def selected(name):
        """--only names ops by their first word; the latency-bound Qwen rows only come with `qwen`."""
        if not only:
            return True
        return "qwen" in only if " qwen " in name else name.split()[0] in only

    def run(r: Row, min_bytes=ROTATION_MIN):
        if not selected(r.name):
            return
        if r.latency:
            sets, rot = [r.make_set(i) for i in range(2)], None
        else:
            sets, rot = rotation(torch, r.make_set, min_bytes)
        if profile_launches > 0:
            for i in range(profile_launches):
                r.fn(sets[i % len(sets)])
            torch.cuda.synchronize()
            del sets
            torch.cuda.empty_cache()
            return
        row = {"op": r.name, "shape": r.shape, "dtype": r.dtype, "cfg": r.cfg}
        if r.latency:  # kernel time filled in from the kernel trace; graph replay and one call meanwhile
            warm(torch, r.fn, sets)
            per, _ = time_launches(torch, r.fn, sets, 0, 20)
            row["graph_us"] = round(time_graph(torch, r.fn, sets) * 1e3, 2)
            row["call_us"] = round(median(per) * 1e3, 2)
            ms = row["graph_us"] * 1e-3
        else:  # throughput: the median of 5 regions of back-to-back launches between one event pair
            # The GPU idles briefly first: a VALU-heavy row (f32 SwiGLU or GELU) leaves it in a lower
            # power state for a while, which slowed the next row's table-lookup kernel by ~5 %; each row's
            # warm-up then brings the GPU to that row's own steady state.
            torch.cuda.synchronize()
            time.sleep(SETTLE_S)
            if clocks is not None and clocks.dir is not None:
                clocks.samples = []
                with clocks:
                    ms = time_regions(torch, r.fn, sets)
                vals = [v for v in clocks.samples if v is not None]
                if vals:
                    row["sclk_mhz"] = median(vals)
            else:
                ms = time_regions(torch, r.fn, sets)
            if ms < SHORT_MS:
                # Python issues a launch in ~10 us: below this the GPU waits on the host between launches,
                # so time the same launches back to back from a replayed HIP graph instead.
                row["event_us"] = round(ms * 1e3, 2)
                ms = time_graph(torch, r.fn, sets)
                row["us_method"] = "HIP graph replay, per launch"
            if r.ref is not None:
                # torch's kernel with the same traffic, timed the same way on the same buffers: where buffers
                # land in HBM moves a streaming kernel by ~2-3 %, and machines differ by a few per cent; this
                # reference shares both with the row.
                label, rfn = r.ref
                rms = time_regions(torch, rfn, sets)
                if rms < SHORT_MS:
                    rms = time_graph(torch, rfn, sets)
                row["torch_ref"], row["torch_ref_us"] = label, round(rms * 1e3, 2)
        gbs = r.alg_bytes / (ms * 1e-3) / 1e9
        row.update({"us": round(ms * 1e3, 2), "GB/s": round(gbs, 1), "pct_peak": round(100 * gbs / PEAK_GBS, 1),
                    f"{r.unit_name}/s": round(r.units / (ms * 1e-3), 1), "alg_bytes": r.alg_bytes,
                    "latency_bound": r.latency})
        if rot is not None:
            row["rotation_bytes"], row["sets"] = rot, len(sets)
        if r.cpu is not None and orc is not None:
            call, sample = r.cpu()
            sec, _ = cpu_time(call, cpu_budget)
            row[f"cpu_{r.unit_name}/s"] = round(sample / sec, 1)
            row["cpu_sample"] = sample
            row["gpu_vs_cpu"] = round((r.units / (ms * 1e-3)) / (sample / sec), 1)
        res.append(row)
        del sets
        torch.cuda.empty_cache()

    # C2: fused add + RMSNorm at Llama-3-8B width, half precision
    rows, dim = 16384, 4096
    for dt, tag in ((f16, "f16"), (bf16, "bf16")):
        w = gen(torch, (dim,), 3, dev, f32, 0.1, 1.0)
        run(Row("add_rms_norm", f"{rows}x{dim}", tag + " (f32 w)", 4 * rows * dim * 2 + dim * 4, rows, "rows",
                lambda i, dt=dt: (gen(torch, (rows, dim), 30 + i, dev, dt), gen(torch, (rows, dim), 40 + i, dev, dt),
                                  torch.empty(rows, dim, device=dev, dtype=dt)),
                lambda s, w=w: ops.add_rms_norm(s[0], s[1], w, 1e-5, out=s[2]),
                lambda: (lambda x=nrm(256, dim), r=nrm(256, dim), w=nrm(dim, scale=0.1, mean=1.0):
                         orc.add_rms_norm(x, r, w, 1e-5), 256), cfg=2))
    # The out-of-place form (the sum to its own buffer, the residual only read), f32 at the headline shape
    w = gen(torch, (dim,), 3, dev, f32, 0.1, 1.0)
    run(Row("add_rms_norm_to", f"{rows}x{dim}", "f32 (f32 w)", 4 * rows * dim * 4 + dim * 4, rows, "rows",
            lambda i: (gen(torch, (rows, dim), 10 + i, dev, f32), gen(torch, (rows, dim), 20 + i, dev, f32),
                       torch.empty(rows, dim, device=dev, dtype=f32), torch.empty(rows, dim, device=dev, dtype=f32)),
            lambda s, w=w: ops.add_rms_norm(s[0], s[1], w, 1e-5, out=s[2], sum_out=s[3]),
            lambda: (lambda x=nrm(256, dim), r=nrm(256, dim), w=nrm(dim, scale=0.1, mean=1.0):
                     orc.add_rms_norm(x, r, w, 1e-5), 256)))
    # Plain RMSNorm at the same width (the norm the fused kernel's second half is)
    for dt, tag in ((f32, "f32"), (f16, "f16"), (bf16, "bf16")):
        w = gen(torch, (dim,), 3, dev, f32, 0.1, 1.0)
        es = 4 if dt == f32 else 2
        run(Row("rms_norm", f"{rows}x{dim}", tag + " (f32 w)", 2 * rows * dim * es + dim * 4, rows, "rows",
                lambda i, dt=dt: (gen(torch, (rows, dim), 20 + i, dev, dt), torch.empty(rows, dim, device=dev, dtype=dt)),
                lambda s, w=w: ops.rms_norm(s[0], w, 1e-5, out=s[1]),
                lambda: (lambda x=nrm(256, dim), w=nrm(dim, scale=0.1, mean=1.0): orc.rms_norm(x, w, 1e-5), 256),
                ref=("torch neg", lambda s: torch.neg(s[0], out=s[1]))))
    # C3: RoPE, Q 32 + K 8 heads, T 8192, head_dim 128, in place
    T, D = 8192, 128
    pos = torch.arange(T, dtype=torch.int32, device=dev)
    for dt, tag in ((f32, "f32"), (f16, "f16")):
        for il in (False, True):
            n_el = (32 + 8) * T * D
            run(Row("rope_" + ("interleaved" if il else "neox"), f"q32+k8 x {T} x {D}", tag,
                    2 * n_el * (4 if dt == f32 else 2), T, "tokens",
                    lambda i, dt=dt: (gen(torch, (1, 32, T, D), 50 + i, dev, dt), gen(torch, (1, 8, T, D), 60 + i, dev, dt)),
                    lambda s, il=il: ops.rope_(s[0], s[1], pos, 5e5, interleaved=il),
                    lambda il=il: (lambda x=nrm(1, 40, 32, D), p=np.arange(4000, 4032):
                                   orc.apply_rope_partial_scaled(x, p, 5e5, D, 1.0, il), 32), cfg=3,
                    ref=("torch _foreach_neg_ (q and k in place, one launch)", lambda s: torch._foreach_neg_([s[0], s[1]]))))
    # C4: SwiGLU [8192, 14336] f16, GELU-tanh [8192, 10240] f16
    n = 8192 * 14336
    for dt, tag, es, seed in ((f16, "f16", 2, 70), (f32, "f32", 4, 75)):
        run(Row("swiglu", "8192x14336", tag, 3 * n * es, 8192, "rows",
                lambda i, dt=dt, seed=seed: (gen(torch, (8192, 14336), seed + i, dev, dt, 2.0),
                                             gen(torch, (8192, 14336), seed + 10 + i, dev, dt, 2.0),
                                             torch.empty(8192, 14336, device=dev, dtype=dt)),
                lambda s: ops.swiglu(s[0], s[1], out=s[2]),
                lambda: (lambda g=nrm(64, 14336, scale=2.0), u=nrm(64, 14336, scale=2.0): orc.swiglu(g, u), 64),
                cfg=4 if dt == f16 else None, ref=("torch mul", lambda s: torch.mul(s[0], s[1], out=s[2]))))
    if profile_launches == 0 or not only or "gelu_tanh" in only or "gelu_erf" in only:
        ops.init(dev)
    n = 8192 * 10240
    # f32 is the reference's own activation type (glibc's tanhf per element)
    for dt, tag, es, seed in ((f16, "f16", 2, 90), (f32, "f32", 4, 95)):
        run(Row("gelu_tanh", "8192x10240", tag, 2 * n * es, 8192, "rows",
                lambda i, dt=dt, seed=seed: (gen(torch, (8192, 10240), seed + i, dev, dt, 2.0),
                                             torch.empty(8192, 10240, device=dev, dtype=dt)),
                lambda s: ops.gelu_tanh(s[0], out=s[1]),
                lambda: (lambda x=nrm(64, 10240, scale=2.0): orc.gelu(x), 64), cfg=4 if dt == f16 else None,
                ref=("torch neg", lambda s: torch.neg(s[0], out=s[1]))))
    # LayerNorm (+ bias), erf-GELU and the bias add: the encoder-family norm / activation path
    wl, bl = gen(torch, (dim,), 4, dev, f32, 0.1, 1.0), gen(torch, (dim,), 5, dev, f32, 0.1)
    for dt, tag, es in ((f32, "f32", 4), (f16, "f16 (f32 w,b)", 2)):
        run(Row("layer_norm", f"{rows}x{dim}", tag, 2 * rows * dim * es + 2 * dim * 4, rows, "rows",
                lambda i, dt=dt: (gen(torch, (rows, dim), 150 + i, dev, dt, 2.0, 0.5),
                                  torch.empty(rows, dim, device=dev, dtype=dt)),
                lambda s: ops.layer_norm(s[0], wl, bl, 1e-5, out=s[1]),
                lambda: (lambda x=nrm(256, dim, scale=2.0, mean=0.5), w=nrm(dim, scale=0.1, mean=1.0),
                         b=nrm(dim, scale=0.1): orc.layer_norm(x, w, b, 1e-5), 256),
                ref=("torch neg", lambda s: torch.neg(s[0], out=s[1]))))
    run(Row("add_bias", f"{rows}x{dim}", "f32", 2 * rows * dim * 4 + dim * 4, rows, "rows",
            lambda i: (gen(torch, (rows, dim), 160 + i, dev, f32), torch.empty(rows, dim, device=dev)),
            lambda s: ops.add_bias(s[0], bl, out=s[1]),
            lambda: (lambda y=nrm(256, dim), b=nrm(dim, scale=0.1): orc.add_bias_last_dim(y, b), 256),
            ref=("torch add (broadcast bias)", lambda s: torch.add(s[0], bl, out=s[1]))))
    n = 12000 * 5120
    for dt, tag, es in ((f32, "f32", 4), (f16, "f16", 2)):
        run(Row("gelu_erf", "12000x5120", tag, 2 * n * es, 12000, "rows",
                lambda i, dt=dt: (gen(torch, (12000, 5120), 170 + i, dev, dt, 2.0),
                                  torch.empty(12000, 5120, device=dev, dtype=dt)),
                lambda s: ops.gelu_erf(s[0], out=s[1]),
                lambda: (lambda x=nrm(64, 5120, scale=2.0): orc.gelu_erf(x), 64),
                ref=("torch neg", lambda s: torch.neg(s[0], out=s[1]))))
    # Decode-chain helpers: head transpose of a Llama-3-8B prefill Q, KV-cache append of its K
    T, H, D = 8192, 32, 128
    for dt, tag, es in ((f32, "f32", 4), (f16, "f16", 2)):
        run(Row("transpose_heads", f"{T}x{H}x{D}", tag, 2 * T * H * D * es, T, "tokens",
                lambda i, dt=dt: (gen(torch, (T, H, D), 180 + i, dev, dt), torch.empty(H, T, D, device=dev, dtype=dt)),
                lambda s: ops.transpose_heads(s[0], out=s[1]),
                lambda es=es: (lambda x=(nrm(64, H, D) if es == 4 else
                                         crng.integers(0, 65536, (64, H, D), dtype=np.uint16)):
                               orc.transpose_heads(x, 64, H, D), 64),
                ref=("torch copy_ of the transposed view", lambda s: s[1].copy_(s[0].transpose(0, 1)))))
    run(Row("kv_append", f"8x{T}x{D} -> cache 8x{T}x{D}", "f32->f16", 8 * T * D * (4 + 2), T, "tokens",
            lambda i: (gen(torch, (8, T, D), 190 + i, dev, f32), torch.empty(8, T, D, device=dev, dtype=f16)),
            lambda s: ops.kv_append(s[0], s[1], 0),
            lambda: (lambda x=nrm(8, 64, D), c=np.zeros((8, T, D), np.uint16):
                     orc.kv_append(x, c, L.F16, 8, 64, D, T, 0), 64),
            ref=("torch copy_ f32 -> f16", lambda s: s[1].copy_(s[0]))))
    # The trait path's cache update on a full cache (decode step past 8192 positions): the window
    # slides one row — every head's 8191 kept rows move down (read + write) — then the new row lands.
    run(Row("kv_cache_update", f"8x1x{D} -> full cache 8x{T}x{D}", "f32->f16",
            2 * 8 * (T - 1) * D * 2 + 8 * D * (4 + 2), 1, "tokens",
            lambda i: (gen(torch, (8, 1, D), 210 + i, dev, f32), gen(torch, (8, T, D), 220 + i, dev, f16)),
            lambda s: ops.kv_cache_update(s[0], s[1], T),
            lambda: (lambda x=nrm(8, 1, D), c=np.zeros((8, T, D), np.uint16):
                     orc.kv_cache_update(x, c, L.F16, 8, 1, D, T, T), 1)))
    # The same step into a second cache (the caller then uses it as its cache): each kept row moves once.
    run(Row("kv_cache_update_into", f"8x1x{D} -> full cache 8x{T}x{D}", "f32->f16",
            2 * 8 * (T - 1) * D * 2 + 8 * D * (4 + 2), 1, "tokens",
            lambda i: (gen(torch, (8, 1, D), 210 + i, dev, f32), gen(torch, (8, T, D), 220 + i, dev, f16),
                       torch.empty(8, T, D, device=dev, dtype=f16)),
            lambda s: ops.kv_cache_update_into(s[0], s[1], s[2], T),
            lambda: (lambda x=nrm(8, 1, D), c=np.zeros((8, T, D), np.uint16):
                     orc.kv_cache_update(x, c, L.F16, 8, 1, D, T, T), 1)))

    def cpu_gather(dt, block, nbytes, d_off, nd, hidden, n):
        """The oracle's gather of n ids from a 2048-row table of the same format (cost per row does not
        depend on vocab)."""
        vocab_c = 2048
        nb_c = vocab_c * hidden // block
        t = crng.integers(0, 256, (nb_c, nbytes), dtype=np.uint8)
        if nd:
            t[:, d_off:d_off + 2 * nd] = crng.uniform(0.0005, 0.02, (nb_c, nd)).astype(np.float16).view(np.uint8)
        ids_c = crng.integers(0, vocab_c, n).astype(np.uint32)
        return (lambda: orc.embed_tokens(t, dt, vocab_c, hidden, ids_c)), n

    # C5 and the other table formats: 128256 x 4096 tables, 65536 ids. Each buffer set is a table of
    # its own, an id set of its own and an output, so no launch reads rows the previous one left in cache.
    vocab, hidden, n_ids = 128256, 4096, 65536
    g = torch.Generator(device=dev).manual_seed(7)
    rng = np.random.default_rng(8)
    p = 1.0 / np.arange(1, vocab + 1) ** 1.1
    cdf = np.cumsum(p / p.sum())

    def zipf_ids(i):
        prng = np.random.default_rng(80 + i)
        return prng.permutation(vocab)[np.minimum(np.searchsorted(cdf, prng.random(n_ids)), vocab - 1)]

    formats = ((L.Q4_K, "q4_k", 256, 144, 0, 2), (L.Q8_0, "q8_0", 32, 34, 0, 1), (L.Q4_0, "q4_0", 32, 18, 0, 1),
               (L.Q5_K, "q5_k", 256, 176, 0, 2), (L.Q6_K, "q6_k", 256, 210, 208, 1))
    for dt, name, block, nbytes, d_off, nd in formats:
        dists = ("uniform", "zipf1.1") if dt == L.Q4_K else ("uniform",)
        for dist in dists:
            def make_set(i, dist=dist, block=block, nbytes=nbytes, d_off=d_off, nd=nd):
                ids_np = zipf_ids(i) if dist == "zipf1.1" else rng.integers(0, vocab, n_ids)
                return (q_table(torch, dev, g, vocab, hidden, block, nbytes, d_off, nd),
                        torch.from_numpy(ids_np.astype(np.int32)).to(dev), torch.empty(n_ids, hidden, device=dev))
            row_bytes = hidden // block * nbytes
            run(Row(f"embed_{name} {dist}", f"{vocab}x{hidden} -> {n_ids} ids", f"{name}->f32",
                    n_ids * (row_bytes + 4 + hidden * 4), n_ids, "rows", make_set,
                    lambda s, dt=dt: ops.embed(s[0], dt, vocab, hidden, s[1], out=s[2]),
                    lambda dt=dt, block=block, nbytes=nbytes, d_off=d_off, nd=nd:
                        cpu_gather(dt, block, nbytes, d_off, nd, hidden, 1024), cfg=5 if dt == L.Q4_K else None))
    # C1: Qwen2.5-0.5B layer ops (latency-bound, reported only)
    lrows, tq, vocab_q = latency_rows(torch, ops, dev, orc, nrm, cpu_gather)
    first_latency = len(res)
    for r in lrows:
        run(r)
    if profile_launches == 0 and kernel_trace and any(selected(r.name) for r in lrows):
        times, note = latency_kernel_times([r.name for r in lrows])
        for row in res[first_latency:]:
            if times is not None and row["op"] in times:
                us, kernel = times[row["op"]]
                lr = next(r for r in lrows if r.name == row["op"])
                gbs = lr.alg_bytes / (us * 1e-6) / 1e9
                row.update({"us": round(us, 2), "GB/s": round(gbs, 1), "pct_peak": round(100 * gbs / PEAK_GBS, 1),
                            f"{lr.unit_name}/s": round(lr.units / (us * 1e-6), 1), "kernel": kernel})
                if "cpu_sample" in row:
                    row["gpu_vs_cpu"] = round((lr.units / (us * 1e-6)) / row[f"cpu_{lr.unit_name}/s"], 1)
            row["us_method"] = note if times is not None else f"graph replay per launch ({note})"
    # Device-resident decode engine at Qwen2.5-0.5B shape (24 layers, 896 hidden, 14 + 2 heads x 64,
    # 4864 intermediate, f16 KV cache, Q8_0 embedding): this library's part of a token
    # (projections / attention skipped), launched eagerly and replayed from a HIP graph.
    if profile_launches == 0 and (not only or "engine" in only):
        res.extend(engine_rows(torch, dev, tq, vocab_q))
    return res


class ClockSampler:
    """The GPU's engine clock as the driver reports it (sysfs pp_dpm_sclk, the level marked current),
    sampled every millisecond on a thread while a timed region runs; plus the memory clock and the board power
    cap, read once. Machines differ by a few per cent in speed: this is the clock they ran at."""

    def __init__(self, torch):
        import ctypes
        self.dir = None
        self.samples = []
        try:
            hip = ctypes.CDLL("libamdhip64.so")
            buf = ctypes.create_string_buffer(64)
            if hip.hipDeviceGetPCIBusId(buf, 64, torch.cuda.current_device()) == 0:
                d = Path("/sys/bus/pci/devices") / buf.value.decode().lower()
                if (d / "pp_dpm_sclk").exists():
                    self.dir = d
        except OSError:
            pass

    @staticmethod
    def _current(text):
        for line in text.splitlines():
            if line.rstrip().endswith("*"):
                m = re.search(r"(\d+)\s*Mhz", line, re.I)
                return int(m.group(1)) if m else None
        return None

    def __enter__(self):
        import threading
        self._stop = threading.Event()

        def run():
            while not self._stop.wait(0.001):
                try:
                    self.samples.append(self._current((self.dir / "pp_dpm_sclk").read_text()))
                except OSError:
                    return
        self._t = threading.Thread(target=run, daemon=True) if self.dir else None
        if self._t:
            self._t.start()
        return self

    def __exit__(self, *exc):
        if self._t:
            self._stop.set()
            self._t.join()

    def report(self):
        if self.dir is None:
            return None
        out = {"sclk_mhz_during_headline": None, "samples": len(self.samples)}
        vals = [v for v in self.samples if v is not None]
        if vals:
            out["sclk_mhz_during_headline"] = {"median": median(vals), "min": min(vals), "max": max(vals)}
        for name, f in (("sclk_levels", "pp_dpm_sclk"), ("mclk", "pp_dpm_mclk")):
            try:
                out[name] = " ".join((self.dir / f).read_text().split())
            except OSError:
                out[name] = None
        caps = sorted(self.dir.glob("hwmon/hwmon*/power1_cap"))
        try:
            out["power_cap_w"] = round(int(caps[0].read_text()) / 1e6) if caps else None
        except (OSError, ValueError):
            out["power_cap_w"] = None
        return out


def plain_copy(torch, dev, warmup, steps):
    """This machine's streaming speed, for reading the headline across machines (MI355X machines differ by a few per
    cent): torch's `neg` (a kernel this library did not write) over the headline's byte count, 512 MiB read
    and 512 MiB written per launch, timed like the headline right after it."""
    n = 2 * 16384 * 4096
    sets = [(gen(torch, (n,), 90 + i, dev, torch.float32), torch.empty(n, device=dev)) for i in range(2)]
    ms, _ = time_region(torch, lambda s: torch.neg(s[0], out=s[1]), sets, warmup, steps)
    gbs = 2 * n * 4 / (ms / steps * 1e-3) / 1e9
    del sets
    torch.cuda.empty_cache()
    return {"kernel": "torch neg, 2 x 16384 x 4096 f32 (read + write)", "GB/s": round(gbs, 1),
            "pct_peak": round(100 * gbs / PEAK_GBS, 1)}


def calibration_copies(torch, ops, dev, warmup, steps):
    """Copies of known size for the HBM counters (2 x 16384 x 4096 f32 = 512 MiB read and 512 MiB
    written per launch): torch's `copy_` and `neg` (kernels this library did not write), then the
    library's own element-wise add of a length-1 zero operand."""
    n = 2 * 16384 * 4096
    a = [gen(torch, (n,), 90 + i, dev, torch.float32) for i in range(2)]
    o = [torch.empty(n, device=dev) for _ in range(2)]
    zero = torch.zeros(1, device=dev)
    time_launches(torch, lambda i: o[i].copy_(a[i]), [0, 1], warmup, steps)
    time_launches(torch, lambda i: torch.neg(a[i], out=o[i]), [0, 1], warmup, steps)
    time_launches(torch, lambda i: ops.add(a[i], zero, out=o[i]), [0, 1], warmup, steps)
    return {"copy_bytes_read": n * 4, "copy_bytes_written": n * 4,
            "calibration_kernels": ["torch copy_", "torch neg", "sph add (a + 0)"]}


def host_tensor_rate():
    """The C++ trait mirror's host-tensor rate (tests/native/bench_host_tensor, built by build()): the
    fused add + RMSNorm at the headline shape on host tensors, the host link crossed both ways as the
    reference's trait calls do. Runs as a child process in its own group; returns its JSON object, or
    a dict naming why there is none."""
    exe = ROOT / "tests" / "native" / "_build" / "bench_host_tensor"
    if not exe.exists():
        return {"skipped": "tests/native/_build/bench_host_tensor not built"}
    child = subprocess.Popen([str(exe)], stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True,
                             start_new_session=True)
    try:
        out, _ = child.communicate(timeout=120)
    except subprocess.TimeoutExpired:
        os.killpg(child.pid, signal.SIGKILL)
        child.communicate()
        return {"skipped": "host-tensor child timed out"}
    for ln in out.splitlines():
        if ln.startswith('{"host_tensor"'):
            return json.loads(ln)["host_tensor"]
    return {"skipped": f"host-tensor child failed (rc {child.returncode})"}


def reap_children() -> int:
    """Child processes of this run still alive (there should be none: the kernel-trace child is waited
    for); any found are terminated and waited for, so none outlives bench.py. Returns how many were found."""
    import psutil
    kids = psutil.Process().children(recursive=True)
    for k in kids:
        try:
            k.terminate()
        except psutil.NoSuchProcess:
            pass
    psutil.wait_procs(kids, timeout=5)
    return len(kids)


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), or the platform's processor string."""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown CPU"


# Keys of an op-table row kept in the final line's compact form (the full rows go to the line before it).
COMPACT = ("op", "shape", "dtype", "us", "GB/s", "pct_peak", "graph_us", "rotation_bytes", "gpu_vs_cpu", "sclk_mhz",
           "torch_ref_us")


def compact(row: dict) -> dict:
    """A configuration row as the final line carries it: identity, kernel time, bandwidth, % of peak, the
    bytes its buffers rotate through (throughput rows) or its graph-replay time (latency rows), and the
    GPU/CPU rate ratio."""
    out = {k: row[k] for k in COMPACT if k in row and row[k] is not None}
    out["cfg"] = row["cfg"]
    return out


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: every op here is row- or token-independent, so a multi-GPU run is "
              "N copies of the one-GPU kernel on 1/N of the rows (no exchange step). Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)
    if args.latency_child:
        latency_child()
        return
    import torch

    import sapient_amd
    import sapient_amd.ops as ops

    if not sapient_amd.LIB_PATH.exists():
        from sapient_amd import build
        build.build(verbose=False)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    if args.profile_run and args.only:
        # Launch the selected op-table rows (warmup + steps launches each), then the calibration copies.
        op_table(torch, ops, dev, set(args.only.split(",")), 0.0, profile_launches=args.warmup + args.steps)
        cal = calibration_copies(torch, ops, dev, args.warmup, args.steps)
        print(json.dumps({"profile_run": True, "ops": args.only, "launches_per_row": args.warmup + args.steps, **cal}))
        return
    clocks = ClockSampler(torch)
    rows, dim, alg_bytes, region_ms, wall, rot_bytes = headline(torch, ops, dev, args, clocks)
    if args.profile_run:
        cal = calibration_copies(torch, ops, dev, args.warmup, args.steps)
        print(json.dumps({"profile_run": True, "headline_avg_us": round(region_ms / args.steps * 1e3, 2),
                          "headline_alg_bytes": alg_bytes, **cal}))
        return
    avg_ms = region_ms / args.steps
    achieved = alg_bytes / (avg_ms * 1e-3) / 1e9
    value = alg_bytes * args.steps / (region_ms * 1e-3) / 1e9
    plain = plain_copy(torch, dev, args.warmup, args.steps)

    cpu = None
    if not args.no_cpu:
        import oracle
        n_rows = 2048  # an eighth of the rows; repeated for the time budget
        rng = np.random.default_rng(0)
        xs = rng.standard_normal((n_rows, dim), dtype=np.float32)
        rs = rng.standard_normal((n_rows, dim), dtype=np.float32)
        ws = (rng.standard_normal(dim, dtype=np.float32) * np.float32(0.1) + np.float32(1.0))
        sec, reps = cpu_time(lambda: oracle.add_rms_norm(xs, rs, ws, 1e-5), args.cpu_seconds)
        sample_bytes = 4 * n_rows * dim * 4 + dim * 4
        cpu = {"value": round(sample_bytes / sec / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
               "sample": f"oracle add_rms_norm on {n_rows}x{dim} f32 rows (1/8 of the workload), {reps} reps "
                         f"in {args.cpu_seconds:.0f} s, 1 thread of {cpu_model()} ({os.cpu_count()} host cores "
                         f"visible)",
               "rows_per_s": round(n_rows / sec, 1)}

    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(avg_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded torch.randn ~N(0,1) inputs/residual, weight ~N(1,0.1); torch.Generator "
                "seeds: x 10 and 11, residual 20 and 21 (two rotating sets), weight 3)",
        "config": {"workload": "fused residual-add + RMSNorm, Llama-3-8B width", "rows": rows, "dim": dim,
                   "eps": 1e-5, "io": "x, residual in; normed + updated residual out (f32)",
                   "rows_per_s": round(rows / (avg_ms * 1e-3), 1), "pct_of_peak": round(100 * value / PEAK_GBS, 1)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / PEAK_GBS, 4), "traffic": committed_traffic("add_rms_norm_f32_16384x4096"),
                     "kernel": HEADLINE_KERNEL, "alg_bytes_per_launch": alg_bytes,
                     "avg_launch_us": round(avg_ms * 1e3, 2)},
        "cpu_baseline": cpu,
        "plain_copy": plain,
        "device_clock": clocks.report(),
        "timing": {"region_ms": round(region_ms, 3), "host_wall_ms": round(wall * 1e3, 3),
                   "rotation_bytes": rot_bytes,
                   "method": "one HIP event pair around the timed launches on their stream"},
    }
    if not args.no_ops:
        only = set(args.only.split(",")) if args.only else None
        rows = op_table(torch, ops, dev, only, 0.0 if args.no_cpu else args.op_cpu_seconds,
                        kernel_trace=not args.no_kernel_trace, clocks=ClockSampler(torch))
        # Every row in full on a line of its own, before the final line; the final line keeps the rows of
        # the five benchmark configurations in compact form.
        extra = {"ops_full": rows}
        if not args.no_cpu:
            extra["ops_cpu"] = ("cpu_*/s: the oracle (the reference's algorithm restated in C, f32, one thread) on "
                                "cpu_sample rows / tokens / ids of each shape, timed on this host; gpu_vs_cpu = the "
                                "ratio of the two rates")
        print(json.dumps(extra), flush=True)
        line["ops"] = [compact(r) for r in rows if r.get("cfg") is not None]
        line["ops_note"] = ("rows of configurations 1-5; us = kernel time (latency rows: rocprofv3 kernel trace "
                            "median, beside graph_us per replayed launch), pct_peak of 8 TB/s, gpu_vs_cpu = rate "
                            "over the one-thread oracle's; every row in full on the line before")
    if not args.no_host_tensor:
        line["host_tensor"] = host_tensor_rate()
    line["children_left"] = reap_children()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
