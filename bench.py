#!/usr/bin/env python3
"""Benchmark of the minicompiler HIP backend on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload mlp|gelu|batchnorm|gemm_fp32|gemm_bf16]

A step is one enqueue of the compiled graph (every kernel of one forward
pass over one batch of synthetic, seeded input already resident in HBM).
The headline workload is BASELINE config 2, the fp32 MLP block
(mlp_gelu.mcg) at B=8192: GEMM with bias+GELU fused into its store, GEMM
with bias+residual fused into its store. The other configurations run
first (each after WARM_SECONDS of its own work). The headline then times
each of its launches alone (after WARM_SECONDS of its own steps; back to
back between one pair of HIP events on the executable's stream), then runs
W untimed steps and K timed steps: the K steps find the GPU at the clock it
holds under this work, whatever W is (it idles while the graph compiles and
its buffers upload, and takes 30-40 ms of work to come back). The K steps
are timed between two HIP events on the executable's stream and are issued
by one library call (mc_enqueue_steps), so no per-step Python work sits in
the timed region. GEMM operator rows are timed from a captured HIP
graph of back-to-back launches over rotating operand sets (no host launch
cost; the reference times its GEMMs from a graph, bench_cuda.cpp:445-493).
Every configuration rotates over buffer sets whose footprint exceeds twice
the 256 MB MALL, so no timed launch reads operands the last one left on
chip. The other configurations time at least MIN_TIMED_MS of GPU work per
timed loop (more steps than K when K would run less; `timed_steps` and
`timed_launches` give the counts); the headline times exactly K steps.

Prints ONE JSON line on stdout (below SUMMARY_MAX_BYTES: headline fields,
roofline, cpu_baseline and a short entry per config) and writes the full
record, with every config's detail, to --out. `value` is the step's GEMM throughput (TFLOP/s = the
two GEMMs' 2MNK FLOPs per step / ms_per_step). `roofline` is for the
kernel that takes the most time; `kernels` lists every launch with its
algorithmic work, achieved rate and fraction of the MI355X peak (HBM 8 TB/s;
FP32 matrix 157.3 TFLOP/s; dense bf16/fp16 2.5 PFLOP/s). `configs` adds the
other BASELINE configs measured in the same process (skip with --quick),
each with a `cpu_baseline`: the CPU oracle (a C++ restatement of the
reference's Eigen backend, test infrastructure) on a bounded row sample of
that workload on this host, one thread (the reference's configuration) and
the host's CPU share. `device.clocks` summarises the engine clock (AMD SMI)
while the headline workload ran on the GPU (its warm-up, per-launch timings
and timed steps), one value per firmware snapshot of the metrics table (about
one a second), `device.clocks_timed_steps` the snapshots seen during the
timed steps alone.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import threading
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_HBM_GBS = 8000.0
PEAK_FP32_TFLOPS = 157.3
PEAK_BF16_TFLOPS = 2500.0
METRIC = "fused-kernel HBM GB/s + GEMM TFLOPS, % of MI355X roofline, 1 GPU"
MALL_BYTES = 256 << 20
# Warm-up time of every configuration other than the headline step (which
# runs exactly --warmup untimed steps).
WARM_SECONDS = 0.3
# Every timed loop of the other configs (not the headline, which times
# exactly --steps steps) runs at least this much GPU work (--min-timed-ms):
# loops of about a millisecond read slow on an MI355X, whose clock does not
# hold through short bursts (MLP B=256: 20.9 us per step over 50 steps,
# 18.4-18.6 over 400 or 2000, same process). Runs under rocprofv3 pass 0:
# the many graph replays it adds to the GEMM rows crashed the traced process
# (a host fault after the 8192^3 row, 3 of 3 runs; none without the tracer,
# none under it with 0).
MIN_TIMED_MS = 20.0
# Launches per captured HIP graph in the GEMM rows (replayed as often as the
# timed launches need).
GRAPH_LAUNCHES = 256
# Per-launch and per-GEMM timings are the median of this many runs (their range
# is reported beside them); the headline step time is one run of K steps.
RUNS = 3


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def node_work(graph: dict, launch_nodes=None) -> list[dict]:
    """Algorithmic work of each launch: 2MNK FLOPs for a matmul (also one
    whose store applies a fused elementwise group: it is bound by the matrix
    cores); for an elementwise kernel the bytes of its output plus each
    distinct non-scalar operand read once (the reference's bytes_moved,
    bench/bench_cuda.cpp:79-95). `launch_nodes`: the node ids each launch
    computes (default: one launch per compute node, in id order)."""
    nodes = graph["nodes"]
    if launch_nodes is None:
        launch_nodes = [[n["id"]] for n in nodes if n["op_name"] not in ("input", "const")]
    size = lambda s: int(np.prod(s, dtype=np.int64)) if s else 1
    out = []
    for ids in launch_nodes:
        n = nodes[ids[0]]
        if n["op_name"] == "matmul":
            (m, k), (_, nn) = nodes[n["inputs"][0]]["shape"], nodes[n["inputs"][1]]["shape"]
            out.append({"kind": "gemm", "flop": 2.0 * m * nn * k, "m": m, "n": nn, "k": k, "fused": len(ids) > 1})
        else:
            b = 4 * size(n["shape"])
            for i in sorted(set(n["inputs"])):
                sz = size(nodes[i]["shape"])
                if sz > 1:
                    b += 4 * sz
            out.append({"kind": "elementwise", "bytes": float(b)})
    return out


def rate_entry(name: str, work: dict, ms: float, gemm_peak: float = PEAK_FP32_TFLOPS) -> dict:
    if work["kind"] == "gemm":
        tflops = work["flop"] / (ms * 1e-3) / 1e12
        return {"launch": name, "ms": ms, "flop": work["flop"], "tflops": tflops, "bound": "mfma",
                "peak": gemm_peak, "frac": tflops / gemm_peak}
    gbs = work["bytes"] / (ms * 1e-3) / 1e9
    return {"launch": name, "ms": ms, "bytes": work["bytes"], "gbs": gbs, "bound": "hbm", "peak": PEAK_HBM_GBS,
            "frac": gbs / PEAK_HBM_GBS}


def warm_up_for(seconds: float, batch) -> int:
    """Calls `batch()` (some launches, then a wait for them) until `seconds`
    have passed; returns the number of calls. The GPU raises its clock only
    under sustained load (about 35 ms of back-to-back GEMMs on an MI355X to
    reach a steady clock), so the configurations below warm up for a time,
    as the reference's bench does (bench/bench_cuda.cpp:124-130)."""
    calls, until = 0, time.perf_counter() + seconds
    while time.perf_counter() < until:
        batch()
        calls += 1
    return calls


class ClockSampler:
    """Samples the engine clock (AMD SMI, mc_gpu_clock_sample) every few
    milliseconds on a thread while active, as the reference records the SM
    clock range of a run (bench/harness.hpp:264-279). AMD SMI's value is the
    power-management firmware's snapshot, refreshed about once a second: the
    summary keeps one value per snapshot (by its firmware timestamp), and
    counts the reads apart. A window shorter than the refresh period may see
    no snapshot taken inside it."""

    def __init__(self, mc, period_s: float = 0.002):
        self.mc, self.period = mc, period_s
        self.reads = 0
        self.snapshots: dict[int, float] = {}  # firmware timestamp (ns) -> MHz
        self.samples: list[float] = []  # one per snapshot, in order
        self._stop = threading.Event()
        self._thread = None

    def __enter__(self):
        def run():
            while not self._stop.is_set():
                v, stamp = self.mc.gpu_clock_sample()
                if v > 0:
                    self.reads += 1
                    key = stamp if stamp else -self.reads  # no timestamp: every read counts
                    if key not in self.snapshots:
                        self.snapshots[key] = v
                        self.samples.append(v)
                self._stop.wait(self.period)
        self._thread = threading.Thread(target=run, daemon=True)
        self._thread.start()
        return self

    def __exit__(self, *exc):
        self._stop.set()
        self._thread.join()

    def median(self) -> float:
        x = sorted(self.samples)
        return x[len(x) // 2] if x else 0.0

    def refresh_s(self) -> float | None:
        """Median spacing of the snapshots' firmware timestamps, in seconds."""
        stamps = sorted(k for k in self.snapshots if k > 0)
        gaps = sorted(b - a for a, b in zip(stamps, stamps[1:]))
        return gaps[len(gaps) // 2] / 1e9 if gaps else None

    def summary(self) -> dict:
        x = self.samples
        if not x:
            return {"samples": 0, "reads": self.reads}
        return {"samples": len(x), "reads": self.reads, "min_mhz": min(x), "median_mhz": self.median(),
                "mean_mhz": sum(x) / len(x), "max_mhz": max(x), "snapshot_refresh_s": self.refresh_s()}


def rotation_sets(set_bytes: int) -> int:
    """Buffer sets to cycle so that consecutive launches never find their
    operands in the 256 MB MALL: a footprint above twice its size."""
    return max(1, -(-2 * MALL_BYTES // max(1, set_bytes)) + 1) if set_bytes <= 2 * MALL_BYTES else 1


def steps_for(ms_per_step: float, steps: int, min_ms: float | None) -> int:
    """`steps`, or more when they would run less than min_ms (None:
    MIN_TIMED_MS) of GPU work."""
    min_ms = MIN_TIMED_MS if min_ms is None else min_ms
    if min_ms <= 0:
        return steps
    return max(steps, int(math.ceil(min_ms / max(ms_per_step, 1e-4))))


def time_graph(mc, compiled, steps: int, warmup: int, rotations=None, reps: int | None = None,
               warm_seconds: float = 0.0, sampler: ClockSampler | None = None, launches_first: bool = False,
               min_ms: float | None = None) -> dict:
    """W warmup steps (then more until `warm_seconds` have passed), then K
    steps timed between one pair of HIP events on the executable's stream
    (ms_per_step); the K steps are one mc_enqueue_steps call, whose host time
    per step is reported too. Then each launch of the step alone, `reps`
    times back to back between one pair of HIP events on that stream (its
    mean duration, with no event between launches to perturb it), in RUNS
    runs: the median run, and the range. `rotations`: list of (input_ptrs,
    output_ptrs) bound in turn, so consecutive launches touch different
    buffers (defeats the 256 MB MALL). `sampler` runs during the K steps.

    launches_first: the per-launch timings (after `warm_seconds` of steps)
    come before the W warmup steps and the K timed steps instead of after
    them, so the timed steps run at the clock the GPU holds under this work
    whatever W is (an MI355X takes 30-40 ms of back-to-back work to reach
    it from idle, and idles while the graph is compiled and its buffers are
    uploaded).

    min_ms: when K steps (or `reps` launches) would run less GPU work than
    this (None: MIN_TIMED_MS), more are timed (steps_for, from a timing of
    the warm-up steps); `timed_steps` reports the count. 0 times exactly K
    steps."""
    stream = compiled.stream
    start, stop = mc.Event(), mc.Event()
    given_reps = reps

    def size_loops():
        nonlocal steps, reps
        if (MIN_TIMED_MS if min_ms is None else min_ms) > 0:
            n = max(warmup, 10)
            start.record(stream)
            compiled.enqueue_steps(n, sets=rotations)
            stop.record(stream)
            compiled.synchronize()
            steps = steps_for(start.elapsed_ms(stop) / n, steps, min_ms)
        reps = given_reps or max(steps, 10)

    def extra():
        compiled.enqueue_steps(max(warmup, 10), sets=rotations)
        compiled.synchronize()

    def per_launch():
        launch_ms, launch_range = [], []
        for j in range(compiled.kernel_launches):
            compiled.enqueue_steps(2, launch=j, sets=rotations)
            runs = []
            for _ in range(RUNS):
                start.record(stream)
                compiled.enqueue_steps(reps, launch=j, sets=rotations)
                stop.record(stream)
                compiled.synchronize()
                runs.append(start.elapsed_ms(stop) / reps)
            launch_ms.append(statistics.median(runs))
            launch_range.append([min(runs), max(runs)])
        return launch_ms, launch_range

    if launches_first:
        warm_up_for(warm_seconds, extra)
        size_loops()
        launch_ms, launch_range = per_launch()
    compiled.enqueue_steps(warmup, sets=rotations)
    compiled.synchronize()
    if not launches_first:
        warm_up_for(warm_seconds, extra)
        size_loops()
    if sampler is not None:
        sampler.__enter__()
    t0 = time.perf_counter()
    start.record(stream)
    host_us = compiled.enqueue_steps(steps, sets=rotations)
    stop.record(stream)
    compiled.synchronize()
    wall = time.perf_counter() - t0
    if sampler is not None:
        sampler.__exit__()
    total_ms = start.elapsed_ms(stop)
    if not launches_first:
        launch_ms, launch_range = per_launch()
    return {"total_ms": total_ms, "ms_per_step": total_ms / steps, "timed_steps": steps, "wall_s": wall,
            "host_us_per_step": host_us, "launch_ms": launch_ms, "launch_ms_range": launch_range, "launch_reps": reps,
            "launch_runs": RUNS,
            "order": "per-launch timings, then warmup and timed steps" if launches_first else
                     "warmup and timed steps, then per-launch timings"}


def graph_rotation(mc, compiled, make_inputs) -> tuple[list, list]:
    """Input/output buffer sets of `compiled` (inputs filled by
    make_inputs()) cycled past the MALL; returns (sets, owned buffers)."""
    set_bytes = 4 * (sum(compiled.input_sizes) + sum(compiled.output_sizes))
    n = rotation_sets(set_bytes)
    xs = make_inputs()
    bufs, sets = [], []
    for _ in range(n):
        ins = [mc.DeviceBuffer.from_array(x) for x in xs]
        outs = [mc.DeviceBuffer(4 * m) for m in compiled.output_sizes]
        bufs.append((ins, outs))
        sets.append(([b.ptr for b in ins], [b.ptr for b in outs]))
    return sets, bufs


def bench_mlp(mc, batch: int, steps: int, warmup: int, options=None, warm_seconds: float = 0.0,
              sampler: ClockSampler | None = None, launches_first: bool = False,
              min_ms: float | None = None) -> dict:
    c = mc.Compiled(path=mc.graph_path("mlp_gelu"), dims={"B": batch}, options=options)
    x = mc.uniform(batch * 512, 1, -1.0, 1.0)
    c.upload([x])
    # Graph replay captures once per binding: no rotation for it.
    rot, bufs = (None, None) if options and options.get("graph") else graph_rotation(mc, c, lambda: [x])
    t = time_graph(mc, c, steps, warmup, rot, warm_seconds=warm_seconds, sampler=sampler,
                   launches_first=launches_first, min_ms=min_ms)
    work = node_work(c.graph(), c.launch_nodes)
    names = c.launch_names
    kernels = [rate_entry(n, w, ms) for n, w, ms in zip(names, work, t["launch_ms"])]
    for e, r in zip(kernels, t["launch_ms_range"]):
        e["ms_range"] = r
    flop = sum(w["flop"] for w in work if w["kind"] == "gemm")
    return {"compiled": c, "timing": t, "kernels": kernels, "gemm_flop": flop, "buffer_sets": len(rot) if rot else 1,
            "value": flop / (t["ms_per_step"] * 1e-3) / 1e12, "jit_ms": c.jit_compile_ms, "buffers": bufs}


def bench_elementwise_graph(mc, name: str, dims: dict, make_input, steps: int, warmup: int) -> dict:
    """One fused group, rotating over input/output buffer sets whose total
    footprint exceeds twice the MALL."""
    c = mc.Compiled(path=mc.graph_path(name), dims=dims)
    x = make_input(c.input_sizes[0])
    rot, bufs = graph_rotation(mc, c, lambda: [x])
    t = time_graph(mc, c, steps, warmup, rot, warm_seconds=WARM_SECONDS)
    work = node_work(c.graph(), c.launch_nodes)
    (k,) = [rate_entry(n, w, ms) for n, w, ms in zip(c.launch_names, work, t["launch_ms"])]
    k["ms_range"] = t["launch_ms_range"][0]
    k["gbs_range"] = [k["bytes"] / (ms * 1e-3) / 1e9 for ms in reversed(k["ms_range"])]
    return {"config": name, "dims": dims, "buffer_sets": len(rot), "kernel": k, "ms_per_step": t["ms_per_step"],
            "timed_steps": t["timed_steps"], "launch_reps": t["launch_reps"],
            "host_us_per_step": t["host_us_per_step"], "gbs": k["gbs"], "frac": k["frac"]}


# Child process of bench_copy_ceiling: PyTorch's copy_ of `nbytes` over
# `sets` rotating tensor pairs, after `warm` seconds of copies, timed with
# torch events over at least `min_ms` of copies in `runs` runs (median).
TORCH_COPY_CHILD = r"""
import json, math, statistics, sys, time
import torch
nbytes, sets, warm, min_ms, runs = int(sys.argv[1]), int(sys.argv[2]), float(sys.argv[3]), float(sys.argv[4]), int(sys.argv[5])
if not torch.cuda.is_available():
    sys.exit("torch sees no GPU")
xs = [(torch.empty(nbytes // 4, device="cuda").uniform_(), torch.empty(nbytes // 4, device="cuda")) for _ in range(sets)]
def burst(n):
    for i in range(n):
        x, y = xs[i % sets]
        y.copy_(x)
until = time.perf_counter() + warm
while time.perf_counter() < until:
    burst(20)
    torch.cuda.synchronize()
e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
e0.record(); burst(20); e1.record(); torch.cuda.synchronize()
reps = max(20, int(math.ceil(min_ms / max(e0.elapsed_time(e1) / 20, 1e-4))))
ts = []
for _ in range(runs):
    e0.record(); burst(reps); e1.record(); torch.cuda.synchronize()
    ts.append(e0.elapsed_time(e1) / reps)
ms = statistics.median(ts)
print(json.dumps({"ms": ms, "ms_range": [min(ts), max(ts)], "gbs": 2 * nbytes / (ms * 1e-3) / 1e9,
                  "copies_timed": reps, "torch": torch.__version__}))
"""


def bench_copy_ceiling(mc, steps: int, warmup: int, nbytes: int = 128 << 20) -> dict:
    """Streaming ceilings measured beside the generated kernels: a copy of
    `nbytes` (read once, written once) by (1) the generated copy_neg kernel
    (graphs/copy_neg.mcg, y = -x, the same size), (2) the HIP runtime's own
    device-to-device copy (hipMemcpyAsync, the runtime's blit kernel) and
    (3) PyTorch's copy_, in a child process (TORCH_COPY_CHILD), when torch
    is installed and sees the GPU. Each rotates over buffer
    pairs past the MALL and times at least MIN_TIMED_MS of back-to-back work;
    GB/s counts the bytes read plus the bytes written."""
    out = {"bytes_each_way": nbytes}
    rows = nbytes // (4 * 4096)
    k = bench_elementwise_graph(mc, "copy_neg", {"M": rows, "N": 4096}, lambda n: mc.uniform(n, 1, -1.0, 1.0),
                                steps, warmup)
    out["mc_copy_neg"] = {"ms": k["kernel"]["ms"], "gbs": k["gbs"], "launch": k["kernel"]["launch"]}
    pairs = [(mc.DeviceBuffer(nbytes), mc.DeviceBuffer(nbytes)) for _ in range(rotation_sets(2 * nbytes))]
    for src, _ in pairs:
        src.fill_bytes(0x3c)
    launches = [lambda st, s=s_, d=d_: mc.memcpy_dtod_async(d.ptr, s.ptr, nbytes, st) for s_, d_ in pairs]
    t = time_gemm(mc, launches, 20, 2)
    for mode in ("graph", "direct"):
        out[f"hip_memcpy_dtod_{mode}"] = {"ms": t[mode]["ms"], "gbs": 2 * nbytes / (t[mode]["ms"] * 1e-3) / 1e9}
    del pairs, launches
    # PyTorch ships its own HIP runtime under the same soname; in this
    # process the library's is loaded, so PyTorch runs in a child process.
    import subprocess
    try:
        proc = subprocess.run([sys.executable, "-c", TORCH_COPY_CHILD, str(nbytes), str(rotation_sets(2 * nbytes)),
                               str(WARM_SECONDS), str(MIN_TIMED_MS), str(RUNS)],
                              capture_output=True, text=True, timeout=300)
        res = [json.loads(l) for l in proc.stdout.splitlines() if l.startswith("{")]
        if proc.returncode == 0 and res:
            out["torch_copy_"] = res[-1]
        else:
            out["torch_copy_error"] = (proc.stderr or proc.stdout)[-300:]
    except (OSError, subprocess.TimeoutExpired) as e:
        out["torch_copy_error"] = str(e)[:300]
    return out


def bench_fusion(mc, dims: dict, rounds: int = 40) -> dict:
    """The reference's fusion comparison (bench/bench_cuda.cpp:182-288): the
    GELU chain compiled unfused (passes dne,fold,dne: one launch per op) and
    fused (the default pipeline: one launch), both over buffer sets past the
    MALL, timed in interleaved rounds whose variant order is a fresh seeded
    shuffle each round. A sample is one pair of HIP events around a run of
    steps on the executable's stream (enough steps for about 2 ms of work).
    Time = median over rounds; speed-up = median over rounds of
    unfused/fused in the same round; GB/s = the bytes every launch of the
    variant reads and writes (the reference's bytes_moved) / median time.
    The two variants' outputs must agree first (normwise, within 1e-5)."""
    import random

    x = mc.uniform(int(np.prod(list(dims.values()))), 1, -3.0, 3.0)
    variants = []
    for name, passes in (("unfused", "dne,fold,dne"), ("fused", "default")):
        c = mc.Compiled(path=mc.graph_path("gelu_chain"), dims=dims, passes=passes)
        rot, bufs = graph_rotation(mc, c, lambda: [x])
        work = node_work(c.graph(), c.launch_nodes)
        variants.append({"name": name, "passes": passes, "c": c, "rot": rot, "bufs": bufs,
                         "bytes": sum(w["bytes"] for w in work), "samples": []})
    outs = []
    for v in variants:
        v["c"].upload([x])
        v["c"].enqueue()
        outs.append(v["c"].download()[0].astype(np.float64))
    diff = float(np.max(np.abs(outs[0] - outs[1])) / max(1.0, float(np.max(np.abs(outs[1])))))
    if not diff <= 1e-5:
        raise RuntimeError(f"fused and unfused GELU differ by {diff:g} (normwise)")
    start, stop = mc.Event(), mc.Event()
    for v in variants:
        c = v["c"]
        c.enqueue_steps(10, sets=v["rot"])
        start.record(c.stream)
        c.enqueue_steps(10, sets=v["rot"])
        stop.record(c.stream)
        c.synchronize()
        v["steps"] = max(4, int(math.ceil(2.0 / max(start.elapsed_ms(stop) / 10, 1e-4))))
        warm_up_for(WARM_SECONDS, lambda c=c, v=v: (c.enqueue_steps(v["steps"], sets=v["rot"]), c.synchronize()))
    order = random.Random(20261005)
    for _ in range(rounds):
        for j in order.sample(range(len(variants)), len(variants)):
            v = variants[j]
            c = v["c"]
            start.record(c.stream)
            c.enqueue_steps(v["steps"], sets=v["rot"])
            stop.record(c.stream)
            c.synchronize()
            v["samples"].append(start.elapsed_ms(stop) / v["steps"])
    paired = sorted(u / f for u, f in zip(variants[0]["samples"], variants[1]["samples"]))
    pct = lambda xs, q: xs[min(len(xs) - 1, int(q * len(xs)))]
    out = {"config": "gelu_chain", "dims": dims, "rounds": rounds, "max_normwise_diff": diff,
           "speedup": {"median": statistics.median(paired), "p10": pct(paired, 0.1), "p90": pct(paired, 0.9)}}
    for v in variants:
        ms = statistics.median(v["samples"])
        out[v["name"]] = {"passes": v["passes"], "launches": v["c"].kernel_launches, "bytes_moved": v["bytes"],
                          "ms": ms, "ms_range": [min(v["samples"]), max(v["samples"])],
                          "steps_per_sample": v["steps"], "buffer_sets": len(v["rot"]),
                          "gbs": v["bytes"] / (ms * 1e-3) / 1e9, "frac": v["bytes"] / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS}
        v["c"].close()
        del v["bufs"]
    return out


def time_gemm(mc, launches, steps: int, warmup: int, min_ms: float | None = None) -> dict:
    """Mean duration of one launch, over `steps` back-to-back launches that
    cycle through `launches` (one closure per operand set, each enqueueing
    on the stream it is given), after `warmup` rounds and WARM_SECONDS of
    warm-up; more launches when `steps` would run less than min_ms of GPU
    work (`timed_steps` reports the count). Timed two ways, RUNS runs each
    (median and range): `graph`, a HIP graph of the launches captured once
    and replayed between one pair of HIP events (no host launch cost, the
    reference's GEMM timing); `direct`, the same launches issued one by one
    from the host."""
    s = mc.Stream()
    for _ in range(warmup):
        for f in launches:
            f(s)

    def issue(stream):
        for i in range(steps):
            launches[i % len(launches)](stream)

    def extra():
        issue(s)
        s.synchronize()

    warm_up_for(WARM_SECONDS, extra)
    start, stop = mc.Event(), mc.Event()
    # The graph holds at most GRAPH_LAUNCHES launches and is replayed as many
    # times as the timed launches need.
    replays = 1
    if (MIN_TIMED_MS if min_ms is None else min_ms) > 0:
        start.record(s)
        issue(s)
        stop.record(s)
        s.synchronize()
        want = steps_for(start.elapsed_ms(stop) / steps, steps, min_ms)
        if want > steps:
            steps = min(want, GRAPH_LAUNCHES)
            replays = -(-want // steps)
    g = mc.CapturedGraph(s, issue)
    out = {"timed_steps": steps * replays}
    for mode in ("graph", "direct"):
        runs = []
        for _ in range(RUNS):
            start.record(s)
            for _ in range(replays):
                g.launch() if mode == "graph" else issue(s)
            stop.record(s)
            s.synchronize()
            runs.append(start.elapsed_ms(stop) / (steps * replays))
        out[mode] = {"ms": statistics.median(runs), "ms_range": [min(runs), max(runs)]}
    del g
    return out


def operand_sets(mc, shapes_bytes: list[int], make) -> list:
    """Operand sets (lists of device buffers from make()) enough to defeat the MALL."""
    return [make() for _ in range(rotation_sets(sum(shapes_bytes)))]


def bench_gemm_fp32(mc, cus: int, shapes, steps: int, warmup: int) -> list[dict]:
    out = []
    for m, n, k in shapes:
        kernel = mc.resolve_matmul_kernel("auto", m, n, k, cus)
        splits = mc.matmul_splits(kernel, m, n, k, cus)
        ws_bytes = mc.matmul_workspace_bytes(kernel, m, n, splits)
        a_host, b_host = mc.uniform(m * k, 1, -1.0, 1.0), mc.uniform(k * n, 2, -1.0, 1.0)
        sets = operand_sets(mc, [4 * m * k, 4 * k * n, 4 * m * n, ws_bytes],
                            lambda: (mc.DeviceBuffer.from_array(a_host), mc.DeviceBuffer.from_array(b_host),
                                     mc.DeviceBuffer(4 * m * n), mc.DeviceBuffer(ws_bytes) if ws_bytes else None))
        launches = [lambda st, a=a, b=b, c=c, ws=ws: mc.launch_matmul(kernel, a.ptr, b.ptr, c.ptr, m, n, k, st, splits,
                                                                     ws.ptr if ws else None)
                    for a, b, c, ws in sets]
        t = time_gemm(mc, launches, steps, warmup)
        ms = t["graph"]["ms"]
        flop = 2.0 * m * n * k
        e = {"m": m, "n": n, "k": k, "kernel": kernel, "splits": splits,
             "k_ranges": mc.matmul_k_ranges(kernel, m, n, k, splits), "operand_sets": len(sets), "ms": ms,
             "ms_range": t["graph"]["ms_range"], "timed_launches": t["timed_steps"],
             "timing": "hip graph of back-to-back launches",
             "ms_direct_launches": t["direct"]["ms"], "tflops": flop / (ms * 1e-3) / 1e12}
        e["frac"] = e["tflops"] / PEAK_FP32_TFLOPS
        if m <= 32:  # HBM-bound skinny shape: report bytes too
            byt = 4.0 * (m * k + k * n + m * n)
            e["bytes"] = byt
            e["gbs"] = byt / (ms * 1e-3) / 1e9
            e["frac_hbm"] = e["gbs"] / PEAK_HBM_GBS
        n_sets = len(sets)
        del sets, launches
        # The same product as a one-matmul compiled graph (the library's own
        # path: mcc, the C ABI's mc_compile): narrow-tile split_k products
        # add their K ranges inside the GEMM kernel there.
        gg = mc.Compiled(f"graph gemm\ninput a : f32[{m}, {k}]\ninput b : f32[{k}, {n}]\nc = matmul a, b\n"
                         f"output c\n")
        rot, bufs = graph_rotation(mc, gg, lambda: [a_host, b_host])
        tg = time_graph(mc, gg, steps, warmup, rot, warm_seconds=WARM_SECONDS)
        gms = tg["launch_ms"][0]
        e["graph"] = {"ms": gms, "ms_range": tg["launch_ms_range"][0], "launch": gg.launch_names[0],
                      "tflops": flop / (gms * 1e-3) / 1e12, "buffer_sets": len(rot)}
        if m <= 32:
            e["graph"]["gbs"] = e["bytes"] / (gms * 1e-3) / 1e9
        gg.close()
        del bufs
        log(f"gemm fp32 {m}x{n}x{k} compiled graph ({e['graph']['launch']}): {gms:.4f} ms "
            f"{e['graph']['tflops']:.1f} TFLOP/s")
        if splits > 1 or m <= 32:
            # The same product as a one-matmul graph compiled with autotune=1
            # (split count and tile configuration timed at compile time).
            g = mc.Compiled(f"graph gemm\ninput a : f32[{m}, {k}]\ninput b : f32[{k}, {n}]\nc = matmul a, b\n"
                            f"output c\n", options={"autotune": 1})
            rot, bufs = graph_rotation(mc, g, lambda: [a_host, b_host])
            tg = time_graph(mc, g, steps, warmup, rot, warm_seconds=WARM_SECONDS)
            tms = tg["launch_ms"][0]
            e["autotuned"] = {"ms": tms, "ms_range": tg["launch_ms_range"][0], "kernel": g.matmul_kernels[0],
                              "launch": g.launch_names[0], "tflops": flop / (tms * 1e-3) / 1e12}
            g.close()
            del bufs
            log(f"gemm fp32 {m}x{n}x{k} autotuned ({e['autotuned']['launch']}): {tms:.4f} ms "
                f"{e['autotuned']['tflops']:.1f} TFLOP/s")
        out.append(e)
        log(f"gemm fp32 {m}x{n}x{k} {kernel} splits={splits} ({e['k_ranges']} K ranges ran): {ms:.4f} ms "
            f"{e['tflops']:.1f} TFLOP/s "
            f"(direct launches {t['direct']['ms']:.4f} ms), {n_sets} operand sets")
    return out


def bench_gemm_lowp(mc, shapes, steps: int, warmup: int) -> list[dict]:
    """The bf16/fp16 kernel on 16-bit operands already in HBM, A in each
    layout the library takes: row-major (mc_launch_matmul_lowp) and packed
    (mc_launch_matmul_lowp_packed; the packing, done once per operand set
    outside the timed loop, is what a compiled graph's rounding of A writes)."""
    out = []
    for m, n, k in shapes:
        a32 = mc.DeviceBuffer.from_array(mc.uniform(m * k, 1, -1.0, 1.0))
        b32 = mc.DeviceBuffer.from_array(mc.uniform(k * n, 2, -1.0, 1.0))
        for kernel, dtype in (("tensor_core_bf16", mc.DTYPE_BF16), ("tensor_core_f16", mc.DTYPE_F16)):
            for layout in ("row-major", "packed"):
                packed = layout == "packed"
                a_bytes = mc.packed_a16_bytes(m, k) if packed else 2 * m * k

                def make():
                    a, b = mc.DeviceBuffer(a_bytes), mc.DeviceBuffer(2 * k * n)
                    if packed:
                        mc.convert_pack_a_f32(dtype, a32.ptr, a.ptr, m, k)
                    else:
                        mc.convert_f32(dtype, a32.ptr, a.ptr, m * k)
                    mc.convert_f32(dtype, b32.ptr, b.ptr, k * n)
                    return a, b, mc.DeviceBuffer(4 * m * n)
                sets = operand_sets(mc, [a_bytes, 2 * k * n, 4 * m * n], make)
                run = mc.launch_matmul_lowp_packed if packed else mc.launch_matmul_lowp
                launches = [lambda st, a=a, b=b, c=c: run(kernel, dtype, a.ptr, b.ptr, c.ptr, m, n, k, st)
                            for a, b, c in sets]
                t = time_gemm(mc, launches, steps, warmup)
                ms = t["graph"]["ms"]
                tf = 2.0 * m * n * k / (ms * 1e-3) / 1e12
                out.append({"m": m, "n": n, "k": k, "kernel": kernel, "inputs": "bf16" if dtype == 1 else "fp16",
                            "a_layout": layout, "operand_sets": len(sets), "ms": ms, "ms_range": t["graph"]["ms_range"],
                            "timed_launches": t["timed_steps"], "ms_direct_launches": t["direct"]["ms"], "tflops": tf,
                            "frac": tf / PEAK_BF16_TFLOPS})
                log(f"gemm {kernel} {m}x{n}x{k}, A {layout}: {ms:.3f} ms {tf:.1f} TFLOP/s ({len(sets)} operand sets)")
                del sets, launches
    return out


def bench_lowp_epilogue(mc, shapes, steps: int, warmup: int) -> list[dict]:
    """BASELINE config 5 with its epilogue: matmul_bias_gelu.mcg (y =
    gelu_tanh(x w + bias), fp32 in and out) compiled with the bf16 / fp16
    matrix-core kernel. A step is one launch: it rounds x to 16 bits (w was
    rounded once, at compile time), then runs the GEMM with bias+GELU fused
    into its store. `tflops` counts the GEMM's 2MNK FLOPs over the measured
    step (rounding of x included). The rounding of x alone (the same
    conversion into packed A, `mc_convert_pack_a_f32`, on a copy of x, timed
    the same way) is reported beside it as `round_x_ms`, a separate
    measurement; nothing is subtracted."""
    out = []
    for m, n, k in shapes:
        x = mc.uniform(m * k, 1, -1.0, 1.0)
        for kernel, dtype in (("tensor_core_bf16", mc.DTYPE_BF16), ("tensor_core_f16", mc.DTYPE_F16)):
            c = mc.Compiled(path=mc.graph_path("matmul_bias_gelu"), dims={"M": m, "K": k, "N": n},
                            options={"matmul": kernel})
            rot, bufs = graph_rotation(mc, c, lambda: [x])
            t = time_graph(mc, c, steps, warmup, rot, warm_seconds=WARM_SECONDS)
            names = c.launch_names
            (j,) = [i for i, nm in enumerate(names) if nm.startswith("matmul")]
            launch_ms = t["launch_ms"][j]
            del c, bufs
            pb = mc.packed_a16_bytes(m, k)
            xs = operand_sets(mc, [4 * m * k, pb], lambda: (mc.DeviceBuffer.from_array(x), mc.DeviceBuffer(pb)))
            rounds = [lambda st, a=a, h=h: mc.convert_pack_a_f32(dtype, a.ptr, h.ptr, m, k, st) for a, h in xs]
            round_ms = time_gemm(mc, rounds, steps, warmup)["graph"]["ms"]
            del xs, rounds
            tf = 2.0 * m * n * k / (t["ms_per_step"] * 1e-3) / 1e12
            out.append({"m": m, "n": n, "k": k, "kernel": kernel, "launches": names, "buffer_sets": len(rot),
                        "ms_per_step": t["ms_per_step"], "launch_ms": launch_ms, "round_x_ms": round_ms,
                        "tflops": tf, "frac": tf / PEAK_BF16_TFLOPS})
            log(f"{kernel} {m}x{n}x{k} + bias + gelu: step {t['ms_per_step']:.3f} ms {tf:.1f} TFLOP/s "
                f"(its GEMM launch {launch_ms:.3f} ms; rounding x alone {round_ms:.3f} ms)")
    return out


# ---------------------------------------------------------------- CPU baseline

def cpu_threads() -> int:
    """This GPU's share of the host (at most 16 threads per GPU on the box)."""
    return max(1, min(os.cpu_count() or 1, 16))


def cpu_time(call, seconds: float, min_reps: int = 3) -> tuple[float, int]:
    """The reference's time_cpu (bench/harness.hpp:67-79): one warm-up call,
    then calls until `seconds` have passed (at least min_reps); the median
    call time and the number of calls."""
    call()
    times, until = [], time.perf_counter() + seconds
    while len(times) < min_reps or time.perf_counter() < until:
        t0 = time.perf_counter()
        call()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def sample_rows(full: int, first: int, per_call, target_s: float = 0.25) -> int:
    """Rows of the workload for one CPU call of about target_s: per_call(r)
    runs r rows once; a first call with `first` rows sets the scale."""
    t0 = time.perf_counter()
    per_call(first)
    el = max(time.perf_counter() - t0, 1e-4)
    return int(max(1, min(full, round(first * target_s / el))))


def host_cpu() -> dict:
    """The host's CPU model and logical core count, recorded with every CPU
    baseline (bench/harness.hpp:194-205, 246)."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "hardware_concurrency": os.cpu_count()}


def cpu_entry(per_row_work: float, unit: str, rows: int, full_rows: int, cap_rows: int, call_of, what: str,
              seconds: float) -> dict:
    """One-thread timing of call_of(rows)() and, on this GPU's host share,
    of call_of(rows x threads)() (more rows, so every thread has a share of
    the same size; at most cap_rows), as throughputs of `per_row_work` units
    per row."""
    from oracle import oracle as orc

    out = {}
    threads = cpu_threads()
    for t, r, secs in ((1, rows, seconds), (threads, min(cap_rows, rows * threads), seconds / 2)):
        orc.set_threads(t)
        per, reps = cpu_time(call_of(r), secs)
        out[t] = (per_row_work * r / per / (1e12 if unit == "TFLOP/s" else 1e9), per, reps, r)
    orc.set_threads(1)
    v1, per1, reps1, _ = out[1]
    va, pera, repsa, ra = out[threads]
    return {"value": v1, "unit": unit, "cores": 1, "threads": 1, "kind": "port",
            "sample": f"{what}: rows 0..{rows - 1} of {full_rows}, {reps1} calls, median {per1 * 1e3:.2f} ms/call, "
                      f"oracle/cpu_oracle.cpp + cpu_gemm.cpp (Eigen semantics, own GEMM; Eigen is not on the box), "
                      f"1 thread, {os.cpu_count()} host cores",
            "all_cores": {"value": va, "threads": threads,
                          "sample": f"rows 0..{ra - 1}, {repsa} calls, median {pera * 1e3:.2f} ms/call"},
            "host": host_cpu()}


def cpu_baseline_graph(mc, name: str, dims_of, full_rows: int, row_elems: int, make_input, per_row_work: float,
                       unit: str, first: int, seconds: float) -> dict:
    """The oracle evaluating graph `name` on its first rows (rows are
    independent in every bench graph: elementwise groups and x·W products)."""
    from oracle import oracle as orc

    cache = {}

    def prepared(rows):
        if rows not in cache:
            cache.clear()
            c = mc.Compiled(path=mc.graph_path(name), dims=dims_of(rows), backend="none")
            g = c.graph()
            consts = {nd["id"]: c.constant(nd["id"]) for nd in g["nodes"] if nd["op_name"] == "const"}
            cache[rows] = (g, consts, make_input(rows * row_elems))
        return cache[rows]

    def call_of(rows):
        g, consts, x = prepared(rows)
        return lambda: orc.evaluate(g, consts, [x])

    orc.set_threads(1)
    rows = sample_rows(full_rows, first, lambda r: call_of(r)())
    return cpu_entry(per_row_work, unit, rows, full_rows, full_rows, call_of, f"{name} {dims_of(full_rows)}", seconds)


def cpu_baseline_gemm(mc, m: int, n: int, k: int, seconds: float, what: str = "") -> dict:
    """The oracle's fp32 GEMM (the reference's Eigen CPU backend has no 16-bit
    GEMM; config 5 is checked against, and compared with, its fp32 GEMM) on
    the first rows of A."""
    from oracle import oracle as orc

    b = mc.uniform(k * n, 2, -1.0, 1.0)
    a_rows = min(m, 2048)
    a = mc.uniform(a_rows * k, 1, -1.0, 1.0)
    orc.set_threads(1)
    call_of = lambda r: (lambda: orc.matmul(a[:r * k], b, r, k, n))
    rows = sample_rows(a_rows, min(m, 4), lambda r: call_of(r)())
    return cpu_entry(2.0 * n * k, "TFLOP/s", rows, m, a_rows, call_of, what or f"fp32 gemm {m}x{n}x{k}", seconds)


def cpu_baseline(batch_rows: int, seconds: float) -> dict:
    """The headline's CPU baseline: the oracle on the first `batch_rows` rows
    of the MLP workload, one thread, repeated for about `seconds` (and the
    host's CPU share for half as long). Throughput in the headline unit."""
    import minicompiler_amd as mc

    e = cpu_baseline_graph(mc, "mlp_gelu", lambda r: {"B": r}, 8192, 512, lambda n: mc.uniform(n, 1, -1.0, 1.0),
                           4.0 * 512 * 2048, "TFLOP/s", batch_rows, seconds)
    return e


# The `config.workload` names of the bench line; profiles/traffic.json keys
# its entries "<workload> | <launch>" by them.
BF16_WORKLOAD = ("bf16 gemm 8192^3, bf16 inputs in HBM, A packed (mc_pack_a16's layout; the row-major row is in "
                 "configs) (BASELINE config 5)")


def mlp_workload(batch: int) -> str:
    return f"mlp_gelu B={batch} D=512 H=2048 fp32 (BASELINE config 2)"


def measured_traffic(workload: str, launch: str):
    """HBM bytes per launch of `launch` in `workload`, from the rocprofv3
    FETCH_SIZE and WRITE_SIZE runs summarised in profiles/traffic.json (each
    counter scaled by what it reads for the copy_neg calibration kernel of
    known size), or None when that kernel has not been counted."""
    path = ROOT / "profiles" / "traffic.json"
    if not path.exists():
        return None
    entry = json.loads(path.read_text()).get("kernels", {}).get(f"{workload} | {launch}")
    return None if entry is None else entry["traffic_bytes"]


FP32_SHAPES = [(1024, 1024, 1024), (2048, 2048, 2048), (4096, 4096, 4096), (8192, 8192, 8192), (256, 256, 16384),
               (16, 4096, 4096)]
LOWP_SHAPES = [(8192, 8192, 8192), (4096, 14336, 4096)]


def cpu_baselines(mc, args, cpu_s: float, headline_s: float) -> dict:
    """Every CPU baseline, computed before any GPU timing (the GPU idles
    meanwhile and drops its clock, so this work must not sit between the GPU
    configs and the headline). Keys: config names, ("gemm", m, n, k) and
    ("epilogue", m, n, k); "headline" for the MLP. cpu_s: seconds of
    one-thread work per config (half that on all threads), 0 for none."""
    out = {}
    if cpu_s <= 0:
        return out
    want = lambda w: args.workload == w or (args.workload == "mlp" and not args.quick)
    if want("gelu"):
        out["gelu"] = cpu_baseline_graph(mc, "gelu_chain", lambda r: {"M": r, "N": 4096}, 4096, 4096,
                                         lambda n: mc.uniform(n, 1, -3.0, 3.0), 8.0 * 4096, "GB/s", 16, cpu_s)
    if want("batchnorm"):
        out["batchnorm"] = cpu_baseline_graph(mc, "batchnorm_relu", lambda r: {"R": r, "C": 256}, 200704, 256,
                                              lambda n: mc.normal(n, 1, 0.0, 1.0), 8.0 * 256, "GB/s", 256, cpu_s)
    shapes = set()
    if want("gemm_fp32"):
        shapes |= set(FP32_SHAPES)
    if want("gemm_bf16"):
        shapes |= set(LOWP_SHAPES)
    for m, n, k in sorted(shapes):
        out[("gemm", m, n, k)] = cpu_baseline_gemm(mc, m, n, k, cpu_s)
    if want("gemm_bf16"):
        for m, n, k in LOWP_SHAPES:
            out[("epilogue", m, n, k)] = cpu_baseline_graph(
                mc, "matmul_bias_gelu", lambda r, k=k, n=n: {"M": r, "K": k, "N": n}, m, k,
                lambda cnt: mc.uniform(cnt, 1, -1.0, 1.0), 2.0 * n * k, "TFLOP/s", 2, cpu_s)
    if args.workload == "mlp" and not args.quick:
        # The batch sweep's small batches: the whole batch each (rows of the
        # MLP are independent, but each row reports its own measured batch).
        for b in (256, 1024):
            out[f"mlp_b{b}"] = cpu_baseline_graph(mc, "mlp_gelu", lambda r: {"B": r}, b, 512,
                                                  lambda cnt: mc.uniform(cnt, 1, -1.0, 1.0), 4.0 * 512 * 2048,
                                                  "TFLOP/s", min(b, 64), cpu_s)
    if args.workload == "mlp" and headline_s > 0:
        out["headline"] = cpu_baseline(256, headline_s)
    return out


def run_configs(mc, args, cus: int, line: dict, cpu: dict) -> None:
    """BASELINE's other configs, each with its CPU baseline from `cpu`."""
    cfgs = line.setdefault("configs", {})
    want = lambda w: args.workload == w or (args.workload == "mlp" and not args.quick)
    if (want("gelu") or want("batchnorm")) and not args.no_copy_ceiling:
        cc = bench_copy_ceiling(mc, args.steps, args.warmup)
        cfgs["copy_ceiling_128MiB"] = cc
        log("copy ceiling (128 MiB each way): " + ", ".join(f"{k} {v['gbs']:.0f} GB/s" for k, v in cc.items()
                                                             if isinstance(v, dict)))
    if want("gelu"):
        e = bench_elementwise_graph(mc, "gelu_chain", {"M": 4096, "N": 4096}, lambda n: mc.uniform(n, 1, -3.0, 3.0),
                                    args.steps, args.warmup)
        if "gelu" in cpu:
            e["cpu_baseline"] = cpu["gelu"]
        cfgs["gelu_4096x4096"] = e
        log(f"gelu: {e['gbs']:.0f} GB/s, host {e['host_us_per_step']:.1f} us/step")
        f = bench_fusion(mc, {"M": 4096, "N": 4096})
        cfgs["gelu_fusion_4096x4096"] = f
        log(f"gelu fusion: unfused {f['unfused']['launches']} launches {f['unfused']['ms'] * 1e3:.1f} us "
            f"({f['unfused']['gbs']:.0f} GB/s), fused {f['fused']['launches']} launch {f['fused']['ms'] * 1e3:.1f} us "
            f"({f['fused']['gbs']:.0f} GB/s), speed-up {f['speedup']['median']:.2f}x")
    if want("batchnorm"):
        e = bench_elementwise_graph(mc, "batchnorm_relu", {"R": 200704, "C": 256},
                                    lambda n: mc.normal(n, 1, 0.0, 1.0), args.steps, args.warmup)
        if "batchnorm" in cpu:
            e["cpu_baseline"] = cpu["batchnorm"]
        cfgs["batchnorm_relu_200704x256"] = e
        log(f"batchnorm: {e['gbs']:.0f} GB/s, host {e['host_us_per_step']:.1f} us/step")
    if args.workload == "mlp" and not args.quick:
        # BASELINE config 2's batch sweep: the small batches are timed with
        # direct launches, with hipGraph replay, and with the split count and
        # tile configuration autotuned at compile time (autotune=1). Rows are
        # independent, so the headline's CPU baseline (per row) covers them.
        for b in (256, 1024):
            entry = {}
            for mode, opts in (("direct", None), ("graph_replay", {"graph": 1}), ("autotuned", {"autotune": 1})):
                r = bench_mlp(mc, b, max(args.steps, 50), args.warmup, opts, WARM_SECONDS)
                entry[mode] = {"ms_per_step": r["timing"]["ms_per_step"], "tflops": r["value"],
                               "timed_steps": r["timing"]["timed_steps"],
                               "launches": r["compiled"].kernel_launches, "buffer_sets": r["buffer_sets"],
                               "host_us_per_step": r["timing"]["host_us_per_step"],
                               "launch_ms": r["timing"]["launch_ms"]}
                del r
            if f"mlp_b{b}" in cpu:
                entry["cpu_baseline"] = cpu[f"mlp_b{b}"]
            cfgs[f"mlp_b{b}"] = entry
            log(f"mlp B={b}: direct {entry['direct']['ms_per_step'] * 1e3:.1f} us/step, "
                f"graph replay {entry['graph_replay']['ms_per_step'] * 1e3:.1f} us/step, "
                f"autotuned {entry['autotuned']['ms_per_step'] * 1e3:.1f} us/step")
    if want("gemm_fp32"):
        g = bench_gemm_fp32(mc, cus, FP32_SHAPES, 20, 2)  # plus WARM_SECONDS per shape
        for e in g:
            key = ("gemm", e["m"], e["n"], e["k"])
            if key in cpu:
                e["cpu_baseline"] = cpu[key]
        cfgs["gemm_fp32"] = g
    if want("gemm_bf16"):
        g = bench_gemm_lowp(mc, LOWP_SHAPES, 20, 2)  # plus WARM_SECONDS
        for e in g:
            key = ("gemm", e["m"], e["n"], e["k"])
            if key in cpu:
                e["cpu_baseline"] = cpu[key]
        cfgs["gemm_bf16_fp16"] = g
        ep = bench_lowp_epilogue(mc, LOWP_SHAPES, 20, 2)
        for e in ep:
            key = ("epilogue", e["m"], e["n"], e["k"])
            if key in cpu:
                e["cpu_baseline"] = cpu[key]
        cfgs["gemm_bf16_fp16_bias_gelu"] = ep


# The final stdout line stays below this many bytes (the record a harness
# parses may be only the tail of stdout); everything else goes to --out.
SUMMARY_MAX_BYTES = 6000


def _r(x, nd=4):
    """A float rounded for the summary line (None stays None)."""
    return None if x is None else float(f"{x:.{nd}g}")


def _cpu_short(e: dict | None) -> dict | None:
    if not e:
        return None
    out = {"value": _r(e["value"]), "threads": e.get("threads", 1)}
    if "all_cores" in e:
        out["all_cores"] = _r(e["all_cores"]["value"])
        out["all_threads"] = e["all_cores"]["threads"]
    return out


def summary_configs(cfgs: dict) -> dict:
    """Per config: value, unit and roofline fraction, with the CPU
    baseline's one-thread and all-thread values; detail stays in --out."""
    out = {}
    for name in ("gelu_4096x4096", "batchnorm_relu_200704x256"):
        if name in cfgs:
            e = cfgs[name]
            out[name] = {"value": _r(e["gbs"]), "unit": "GB/s", "frac": _r(e["frac"], 3),
                         "cpu": _cpu_short(e.get("cpu_baseline"))}
    if "copy_ceiling_128MiB" in cfgs:
        out["copy_ceiling_128MiB"] = {k: _r(v["gbs"]) for k, v in cfgs["copy_ceiling_128MiB"].items()
                                      if isinstance(v, dict)}
    if "gelu_fusion_4096x4096" in cfgs:
        f = cfgs["gelu_fusion_4096x4096"]
        out["gelu_fusion_4096x4096"] = {
            "speedup": _r(f["speedup"]["median"]),
            **{v: {"launches": f[v]["launches"], "ms": _r(f[v]["ms"]), "gbs": _r(f[v]["gbs"])}
               for v in ("unfused", "fused")}}
    for b in (256, 1024):
        if f"mlp_b{b}" in cfgs:
            e = cfgs[f"mlp_b{b}"]
            out[f"mlp_b{b}"] = {**{m: {"us": _r(e[m]["ms_per_step"] * 1e3), "value": _r(e[m]["tflops"])}
                                   for m in ("direct", "graph_replay", "autotuned")},
                                "unit": "TFLOP/s", "cpu": _cpu_short(e.get("cpu_baseline"))}
    if "gemm_fp32" in cfgs:
        rows = {}
        for e in cfgs["gemm_fp32"]:
            r = {"value": _r(e["tflops"]), "frac": _r(e["frac"], 3), "graph": _r(e["graph"]["tflops"]),
                 "cpu": _r(e["cpu_baseline"]["value"]) if "cpu_baseline" in e else None}
            if e.get("splits", 1) > 1:
                r["splits"] = [e.get("k_ranges"), e["splits"]]  # K ranges that ran, of the split count asked for
            if "gbs" in e:
                r.update({"gbs": _r(e["gbs"]), "frac_hbm": _r(e["frac_hbm"], 3), "graph_gbs": _r(e["graph"]["gbs"])})
            rows[f"{e['m']}x{e['n']}x{e['k']}"] = r
        out["gemm_fp32"] = {"unit": "TFLOP/s", "rows": rows}
    for key in ("gemm_bf16_fp16", "gemm_bf16_fp16_bias_gelu"):
        if key in cfgs:
            out[key] = {"unit": "TFLOP/s",
                        "rows": {f"{e['kernel'][12:]} {e['m']}x{e['n']}x{e['k']}"
                                 + (" A packed" if e.get("a_layout") == "packed" else ""):
                                 {"value": _r(e["tflops"]), "frac": _r(e["frac"], 3),
                                  "cpu": _r(e["cpu_baseline"]["value"]) if "cpu_baseline" in e else None}
                                 for e in cfgs[key]}}
    return out


def summary_line(full: dict) -> dict:
    """The one JSON line printed on stdout: the headline fields, `roofline`
    (with `traffic`), `cpu_baseline` (short sample), each launch of the
    headline step and one short entry per other config. Guaranteed below
    SUMMARY_MAX_BYTES: optional parts are dropped, largest first, if not."""
    keep = ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better", "scaling",
            "vs_baseline", "dtype", "data", "config", "roofline")
    line = {k: full[k] for k in keep if k in full}
    if "config" in line:
        line["config"] = {k: v for k, v in line["config"].items() if k != "order"}
    if "cpu_baseline" in full:
        c = full["cpu_baseline"]
        line["cpu_baseline"] = {"value": c["value"], "unit": c["unit"], "cores": c["cores"], "kind": c["kind"],
                                "sample": c["sample"][:240]}
        if "all_cores" in c:
            line["cpu_baseline"]["all_cores"] = {"value": c["all_cores"]["value"],
                                                 "threads": c["all_cores"]["threads"]}
    if "kernels" in full:
        line["kernels"] = [{"launch": k["launch"][:60], "ms": _r(k["ms"]),
                            ("tflops" if k["bound"] == "mfma" else "gbs"): _r(k.get("tflops", k.get("gbs"))),
                            "frac": _r(k["frac"], 3)} for k in full["kernels"]]
    if "device" in full:
        d = full["device"]
        line["device"] = {"name": d.get("name"), "cu_count": d.get("cu_count"),
                          "clock_median_mhz": d.get("clocks", {}).get("median_mhz"),
                          "clock_timed_steps_median_mhz": d.get("clocks_timed_steps", {}).get("median_mhz")}
    if full.get("configs"):
        line["configs"] = summary_configs(full["configs"])
    if full.get("full_record"):
        line["full_record"] = full["full_record"]
    for drop in ("configs", "kernels", "device"):
        if len(json.dumps(line)) < SUMMARY_MAX_BYTES:
            break
        line.pop(drop, None)
    return line


def main() -> int:
    global MIN_TIMED_MS
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # About 70 ms of timed work at B=8192; the 300 warmup steps (about 100 ms)
    # keep the GPU at its working clock first.
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=300)
    ap.add_argument("--workload", default="mlp",
                    choices=["mlp", "gelu", "batchnorm", "gemm_fp32", "gemm_bf16", "copy"])
    ap.add_argument("--batch", type=int, default=8192)
    ap.add_argument("--quick", action="store_true", help="headline workload only (no other configs)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="the headline's CPU baseline")
    ap.add_argument("--config-cpu-seconds", type=float, default=1.5, help="each other config's CPU baseline")
    ap.add_argument("--min-timed-ms", type=float, default=MIN_TIMED_MS,
                    help="GPU work per timed loop of the other configs (0 under rocprofv3)")
    ap.add_argument("--no-copy-ceiling", action="store_true",
                    help="skip the copy ceilings beside the elementwise configs (profiling runs)")
    ap.add_argument("--out", default=str(ROOT / "results" / "bench_full.json"),
                    help="file for the full record (every config's detail); '' for none")
    args = ap.parse_args()
    MIN_TIMED_MS = args.min_timed_ms

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU (rows of each GEMM and elementwise group would shard "
              "across GPUs with no exchange, which is not built). Run with --gpus 1.", file=sys.stderr)
        return 2

    import minicompiler_amd as mc

    dev = mc.device_json()
    cus = dev["cu_count"]
    log(f"device: {dev['name']} {dev['arch']} CUs={cus} clock={dev['clock_mhz']} MHz "
        f"(now {dev.get('clock_now_mhz', 0):.0f} MHz)")
    line = {"metric": METRIC, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "data": "synthetic (seeded splitmix64 uniform/normal, "
                                                            "random-init constants of the graph)"}
    cpu_s = 0.0 if args.no_cpu_baseline else args.config_cpu_seconds
    cpu = cpu_baselines(mc, args, cpu_s, 0.0 if args.no_cpu_baseline else args.cpu_seconds)
    log(f"cpu baselines: {len(cpu)} workloads")
    whole = ClockSampler(mc, period_s=0.05)
    with whole:
        run_configs(mc, args, cus, line, cpu)
    cfgs = line.get("configs", {})
    sampler = ClockSampler(mc)
    # The whole headline workload (warm-up, per-launch timings, timed steps):
    # a few timed steps span a few milliseconds, a handful of AMD SMI reads of
    # a metrics table that can lag the clock.
    headline_run = ClockSampler(mc)

    if args.workload == "mlp":
        with headline_run:
            r = bench_mlp(mc, args.batch, args.steps, args.warmup, sampler=sampler, warm_seconds=WARM_SECONDS,
                          launches_first=True, min_ms=0.0)  # exactly --steps timed steps
        ks = r["kernels"]
        dom = max(ks, key=lambda e: e["ms"])
        line.update({"value": r["value"], "unit": "TFLOP/s", "ms_per_step": r["timing"]["ms_per_step"],
                     "dtype": "f32",
                     "config": {"workload": mlp_workload(args.batch),
                                "global_batch": args.batch, "matmul": ",".join(r["compiled"].matmul_kernels),
                                "buffer_sets": r["buffer_sets"], "order": r["timing"]["order"]},
                     "host_us_per_step": r["timing"]["host_us_per_step"]})
        unit = "TFLOP/s" if dom["bound"] == "mfma" else "GB/s"
        achieved = dom["tflops"] if dom["bound"] == "mfma" else dom["gbs"]
        line["roofline"] = {"bound": dom["bound"], "kernel": dom["launch"], "achieved": achieved,
                            "peak": dom["peak"], "unit": unit, "frac": dom["frac"], "traffic": None}
        line["kernels"] = ks
        fused = [k for k in ks if k["bound"] == "hbm"]
        line["fused_gbs"] = sum(k["bytes"] for k in fused) / (sum(k["ms"] for k in fused) * 1e-3) / 1e9 if fused else None
        line["jit_compile_ms"] = r["jit_ms"]
    elif args.workload == "copy":
        # Byte-counter calibration: reads and writes 128 MiB each, known exactly.
        k = bench_elementwise_graph(mc, "copy_neg", {"M": 8192, "N": 4096}, lambda n: mc.uniform(n, 1, -1.0, 1.0),
                                    args.steps, args.warmup)
        line.update({"value": k["gbs"], "unit": "GB/s", "ms_per_step": k["ms_per_step"], "dtype": "f32",
                     "steps": k["timed_steps"],
                     "config": {"workload": "copy_neg (counter calibration)", **k["dims"]},
                     "roofline": {"bound": "hbm", "kernel": k["kernel"]["launch"], "achieved": k["gbs"],
                                  "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": k["frac"], "traffic": None}})
        if not args.quick:
            line.setdefault("configs", {})["copy_ceiling_128MiB"] = bench_copy_ceiling(mc, args.steps, args.warmup)
    elif args.workload in ("gelu", "batchnorm"):
        k = cfgs["gelu_4096x4096" if args.workload == "gelu" else "batchnorm_relu_200704x256"]
        line.update({"value": k["gbs"], "unit": "GB/s", "ms_per_step": k["ms_per_step"], "dtype": "f32",
                     "steps": k["timed_steps"], "config": {"workload": k["config"], **k["dims"]},
                     "roofline": {"bound": "hbm", "kernel": k["kernel"]["launch"], "achieved": k["gbs"],
                                  "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": k["frac"], "traffic": None}})
        if "cpu_baseline" in k:
            line["cpu_baseline"] = k["cpu_baseline"]
    elif args.workload == "gemm_fp32":
        top = cfgs["gemm_fp32"][3]
        line.update({"value": top["tflops"], "unit": "TFLOP/s", "ms_per_step": top["ms"], "dtype": "f32",
                     "config": {"workload": "fp32 gemm 8192^3 (BASELINE config 4)"},
                     "roofline": {"bound": "mfma", "kernel": top["kernel"], "achieved": top["tflops"],
                                  "peak": PEAK_FP32_TFLOPS, "unit": "TFLOP/s", "frac": top["frac"], "traffic": None}})
        if "cpu_baseline" in top:
            line["cpu_baseline"] = top["cpu_baseline"]
    elif args.workload == "gemm_bf16":
        (top,) = [e for e in cfgs["gemm_bf16_fp16"] if e["kernel"] == "tensor_core_bf16" and e["m"] == 8192
                  and e["a_layout"] == "packed"]
        line.update({"value": top["tflops"], "unit": "TFLOP/s", "ms_per_step": top["ms"], "dtype": "bf16",
                     "config": {"workload": BF16_WORKLOAD},
                     "roofline": {"bound": "mfma", "kernel": top["kernel"], "achieved": top["tflops"],
                                  "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s", "frac": top["frac"], "traffic": None}})
        if "cpu_baseline" in top:
            line["cpu_baseline"] = top["cpu_baseline"]

    if "roofline" in line:
        line["roofline"]["traffic"] = measured_traffic(line["config"]["workload"], line["roofline"]["kernel"])
    d = mc.device_json(headline_run.samples)
    line["device"] = {k: d[k] for k in ("name", "arch", "cu_count", "clock_mhz", "mem_clock_mhz", "bus_width_bits")}
    line["device"]["clocks"] = {**headline_run.summary(),
                                "during": "the headline workload's GPU work (warm-up, per-launch timings, timed steps)",
                                "source": "AMD SMI current GFX clock (mean over XCDs), read every 2 ms; one value per "
                                          "firmware snapshot (the metrics table is refreshed about once a second)"}
    line["device"]["clocks_timed_steps"] = {**sampler.summary(), "during": "the headline's timed steps only"}
    line["device"]["clocks_configs"] = {**whole.summary(), "during": "the other configs' GPU work",
                                        "period_ms": 50}
    if "headline" in cpu:
        line["cpu_baseline"] = cpu["headline"]
    if args.out:
        out = Path(args.out)
        out.parent.mkdir(parents=True, exist_ok=True)
        out.write_text(json.dumps(line, indent=1) + "\n")
        line["full_record"] = str(out)
        log(f"full record: {out} ({out.stat().st_size} bytes)")
    print(json.dumps(summary_line(line)), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
