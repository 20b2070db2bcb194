#!/usr/bin/env python3
"""Benchmark of the minicompiler HIP backend on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload mlp|gelu|batchnorm|gemm_fp32|gemm_bf16]

A step is one enqueue of the compiled graph (every kernel of one forward
pass over one batch of synthetic, seeded input already resident in HBM).
The headline workload is BASELINE config 2, the fp32 MLP block
(mlp_gelu.mcg) at B=8192: GEMM, fused bias+GELU, GEMM, fused
bias+residual. W untimed steps, then exactly K timed steps between two HIP
events on the executable's stream (the default W = 300, about 100 ms at
B=8192, brings the GPU to its steady clock: it raises the clock only under
sustained load; every other configuration warms up for WARM_SECONDS of its
own work). Each kernel's duration is then measured
in the same process on the same stream: the launch alone, back to back,
between one pair of HIP events (events between launches would add their own
gaps to short kernels).

Prints ONE JSON line. `value` is the step's GEMM throughput (TFLOP/s = the
two GEMMs' 2MNK FLOPs per step / ms_per_step). `roofline` is for the
kernel that takes the most time; `kernels` lists every launch with its
algorithmic work, achieved rate and fraction of the MI355X peak (HBM 8 TB/s;
FP32 matrix 157.3 TFLOP/s; dense bf16/fp16 2.5 PFLOP/s). `configs` adds the
other BASELINE configs measured in the same process (skip with --quick).
`cpu_baseline` times the CPU oracle (a C++ restatement of the reference's
Eigen backend, test infrastructure) on a bounded row sample of the same
workload on this host.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
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


def time_graph(mc, compiled, steps: int, warmup: int, rotations=None, reps: int | None = None,
               warm_seconds: float = 0.0) -> dict:
    """W warmup steps (then more until `warm_seconds` have passed), then K
    steps timed between one pair of HIP events on the executable's stream
    (ms_per_step). Then each launch of the step alone, `reps` times back to
    back between one pair of HIP events on that stream (its mean duration,
    with no event between launches to perturb it), in RUNS runs: the median
    run, and the range. `rotations`: list of
    (input_ptrs, output_ptrs) bound in turn, so consecutive launches touch
    different buffers (defeats the 256 MB MALL)."""
    def bind(i):
        if rotations:
            ins, outs = rotations[i % len(rotations)]
            compiled.bind_inputs(ins)
            compiled.bind_outputs(outs)

    stream = compiled.stream
    for i in range(warmup):
        bind(i)
        compiled.enqueue()
    compiled.synchronize()

    def extra():
        for i in range(max(warmup, 10)):
            bind(i)
            compiled.enqueue()
        compiled.synchronize()

    warm_up_for(warm_seconds, extra)
    start, stop = mc.Event(), mc.Event()
    t0 = time.perf_counter()
    start.record(stream)
    for i in range(steps):
        bind(i)
        compiled.enqueue()
    stop.record(stream)
    compiled.synchronize()
    wall = time.perf_counter() - t0
    total_ms = start.elapsed_ms(stop)
    reps = reps or max(steps, 10)
    launch_ms, launch_range = [], []
    for j in range(compiled.kernel_launches):
        for i in range(2):
            bind(i)
            compiled.enqueue_launch(j)
        runs = []
        for _ in range(RUNS):
            start.record(stream)
            for i in range(reps):
                bind(i)
                compiled.enqueue_launch(j)
            stop.record(stream)
            compiled.synchronize()
            runs.append(start.elapsed_ms(stop) / reps)
        launch_ms.append(statistics.median(runs))
        launch_range.append([min(runs), max(runs)])
    bind(0)
    return {"total_ms": total_ms, "ms_per_step": total_ms / steps, "wall_s": wall, "launch_ms": launch_ms,
            "launch_ms_range": launch_range, "launch_reps": reps, "launch_runs": RUNS}


def bench_mlp(mc, batch: int, steps: int, warmup: int, options=None, warm_seconds: float = 0.0) -> dict:
    c = mc.Compiled(path=mc.graph_path("mlp_gelu"), dims={"B": batch}, options=options)
    x = mc.uniform(batch * 512, 1, -1.0, 1.0)
    c.upload([x])
    t = time_graph(mc, c, steps, warmup, warm_seconds=warm_seconds)
    work = node_work(c.graph(), c.launch_nodes)
    names = c.launch_names
    kernels = [rate_entry(n, w, ms) for n, w, ms in zip(names, work, t["launch_ms"])]
    for e, r in zip(kernels, t["launch_ms_range"]):
        e["ms_range"] = r
    flop = sum(w["flop"] for w in work if w["kind"] == "gemm")
    return {"compiled": c, "timing": t, "kernels": kernels, "gemm_flop": flop,
            "value": flop / (t["ms_per_step"] * 1e-3) / 1e12, "jit_ms": c.jit_compile_ms}


def bench_elementwise_graph(mc, name: str, dims: dict, make_input, steps: int, warmup: int) -> dict:
    """One fused group, rotating over input/output buffer sets whose total
    footprint exceeds twice the MALL."""
    c = mc.Compiled(path=mc.graph_path(name), dims=dims)
    n_in, n_out = c.input_sizes[0], c.output_sizes[0]
    set_bytes = 4 * (n_in + n_out)
    sets = max(2, -(-2 * MALL_BYTES // set_bytes) + 1)
    x = make_input(n_in)
    bufs = []
    for _ in range(sets):
        bi, bo = mc.DeviceBuffer.from_array(x), mc.DeviceBuffer(4 * n_out)
        bufs.append((bi, bo))
    rot = [([bi.ptr], [bo.ptr]) for bi, bo in bufs]
    t = time_graph(mc, c, steps, warmup, rot, warm_seconds=WARM_SECONDS)
    work = node_work(c.graph(), c.launch_nodes)
    (k,) = [rate_entry(n, w, ms) for n, w, ms in zip(c.launch_names, work, t["launch_ms"])]
    k["ms_range"] = t["launch_ms_range"][0]
    k["gbs_range"] = [k["bytes"] / (ms * 1e-3) / 1e9 for ms in reversed(k["ms_range"])]
    return {"config": name, "dims": dims, "buffer_sets": sets, "kernel": k, "ms_per_step": t["ms_per_step"],
            "gbs": k["gbs"], "frac": k["frac"]}


def time_gemm(mc, launch, steps: int, warmup: int, runs_out: list | None = None) -> float:
    """Mean duration of `steps` back-to-back launches between one pair of HIP
    events on their stream, after `warmup` launches and a warm-up of
    WARM_SECONDS; the median of RUNS such runs (each run's figure appended
    to `runs_out`)."""
    s = mc.Stream()
    for _ in range(warmup):
        launch(s)

    def extra():
        for _ in range(4):
            launch(s)
        s.synchronize()

    warm_up_for(WARM_SECONDS, extra)
    start, stop = mc.Event(), mc.Event()
    runs = []
    for _ in range(RUNS):
        start.record(s)
        for _ in range(steps):
            launch(s)
        stop.record(s)
        s.synchronize()
        runs.append(start.elapsed_ms(stop) / steps)
    if runs_out is not None:
        runs_out.extend(runs)
    return statistics.median(runs)


def bench_gemm_fp32(mc, cus: int, shapes, steps: int, warmup: int) -> list[dict]:
    out = []
    for m, n, k in shapes:
        kernel = mc.resolve_matmul_kernel("auto", m, n, k, cus)
        splits = mc.matmul_splits(kernel, m, n, k, cus)
        a = mc.DeviceBuffer.from_array(mc.uniform(m * k, 1, -1.0, 1.0))
        b = mc.DeviceBuffer.from_array(mc.uniform(k * n, 2, -1.0, 1.0))
        c = mc.DeviceBuffer(4 * m * n)
        ws_bytes = mc.matmul_workspace_bytes(kernel, m, n, splits)
        ws = mc.DeviceBuffer(ws_bytes) if ws_bytes else None
        runs = []
        ms = time_gemm(mc, lambda s: mc.launch_matmul(kernel, a.ptr, b.ptr, c.ptr, m, n, k, s, splits,
                                                       ws.ptr if ws else None), steps, warmup, runs)
        flop = 2.0 * m * n * k
        e = {"m": m, "n": n, "k": k, "kernel": kernel, "splits": splits, "ms": ms, "ms_range": [min(runs), max(runs)],
             "tflops": flop / (ms * 1e-3) / 1e12}
        e["frac"] = e["tflops"] / PEAK_FP32_TFLOPS
        if m == 16:  # HBM-bound skinny shape: report bytes too
            byt = 4.0 * (m * k + k * n + m * n)
            e["gbs"] = byt / (ms * 1e-3) / 1e9
            e["frac_hbm"] = e["gbs"] / PEAK_HBM_GBS
        if splits > 1 or m <= 32:
            # The same product as a one-matmul graph compiled with autotune=1
            # (split count and tile configuration timed at compile time).
            g = mc.Compiled(f"graph gemm\ninput a : f32[{m}, {k}]\ninput b : f32[{k}, {n}]\nc = matmul a, b\n"
                            f"output c\n", options={"autotune": 1})
            g.upload([mc.uniform(m * k, 1, -1.0, 1.0), mc.uniform(k * n, 2, -1.0, 1.0)])
            t = time_graph(mc, g, steps, warmup, warm_seconds=WARM_SECONDS)
            tms = t["launch_ms"][0]
            e["autotuned"] = {"ms": tms, "ms_range": t["launch_ms_range"][0], "kernel": g.matmul_kernels[0],
                              "tflops": flop / (tms * 1e-3) / 1e12}
            g.close()
            log(f"gemm fp32 {m}x{n}x{k} autotuned ({e['autotuned']['kernel']}): {tms:.3f} ms "
                f"{e['autotuned']['tflops']:.1f} TFLOP/s")
        out.append(e)
        log(f"gemm fp32 {m}x{n}x{k} {kernel}: {ms:.3f} ms {e['tflops']:.1f} TFLOP/s")
    return out


def bench_gemm_lowp(mc, shapes, steps: int, warmup: int) -> list[dict]:
    out = []
    for m, n, k in shapes:
        a32 = mc.DeviceBuffer.from_array(mc.uniform(m * k, 1, -1.0, 1.0))
        b32 = mc.DeviceBuffer.from_array(mc.uniform(k * n, 2, -1.0, 1.0))
        for kernel, dtype in (("tensor_core_bf16", mc.DTYPE_BF16), ("tensor_core_f16", mc.DTYPE_F16)):
            a, b = mc.DeviceBuffer(2 * m * k), mc.DeviceBuffer(2 * k * n)
            mc.convert_f32(dtype, a32.ptr, a.ptr, m * k)
            mc.convert_f32(dtype, b32.ptr, b.ptr, k * n)
            c = mc.DeviceBuffer(4 * m * n)
            runs = []
            ms = time_gemm(mc, lambda s: mc.launch_matmul_lowp(kernel, dtype, a.ptr, b.ptr, c.ptr, m, n, k, s),
                           steps, warmup, runs)
            tf = 2.0 * m * n * k / (ms * 1e-3) / 1e12
            out.append({"m": m, "n": n, "k": k, "kernel": kernel, "inputs": "bf16" if dtype == 1 else "fp16",
                        "ms": ms, "ms_range": [min(runs), max(runs)], "tflops": tf, "frac": tf / PEAK_BF16_TFLOPS})
            log(f"gemm {kernel} {m}x{n}x{k}: {ms:.3f} ms {tf:.1f} TFLOP/s")
            del a, b, c
    return out


def bench_lowp_epilogue(mc, shapes, steps: int, warmup: int) -> list[dict]:
    """BASELINE config 5 with its epilogue: matmul_bias_gelu.mcg (y =
    gelu_tanh(x w + bias), fp32 in and out) compiled with the bf16 / fp16
    matrix-core kernel. A step is one launch: it rounds x to 16 bits (w was
    rounded once, at compile time), then runs the GEMM with bias+GELU fused
    into its store; `gemm_epilogue_tflops` counts the GEMM's 2MNK FLOPs over
    that whole launch, the rounding of x included (about 0.1 ms at 8192^2)."""
    out = []
    for m, n, k in shapes:
        for kernel in ("tensor_core_bf16", "tensor_core_f16"):
            c = mc.Compiled(path=mc.graph_path("matmul_bias_gelu"), dims={"M": m, "K": k, "N": n},
                            options={"matmul": kernel})
            c.upload([mc.uniform(m * k, 1, -1.0, 1.0)])
            t = time_graph(mc, c, steps, warmup, warm_seconds=WARM_SECONDS)
            names = c.launch_names
            (j,) = [i for i, nm in enumerate(names) if nm.startswith("matmul")]
            gemm_ms = t["launch_ms"][j]
            tf = 2.0 * m * n * k / (gemm_ms * 1e-3) / 1e12
            out.append({"m": m, "n": n, "k": k, "kernel": kernel, "launches": names,
                        "ms_per_step": t["ms_per_step"], "gemm_epilogue_ms": gemm_ms, "gemm_epilogue_tflops": tf,
                        "frac": tf / PEAK_BF16_TFLOPS, "launch_ms": t["launch_ms"]})
            log(f"{kernel} {m}x{n}x{k} + bias + gelu: step {t['ms_per_step']:.3f} ms, fused GEMM launch "
                f"{gemm_ms:.3f} ms {tf:.1f} TFLOP/s")
            del c
    return out


def cpu_baseline(batch_rows: int, seconds: float) -> dict:
    """The CPU oracle (restating the reference's Eigen backend) on the first
    `batch_rows` rows of the MLP workload, one thread, repeated for about
    `seconds`. Throughput in the headline unit."""
    import minicompiler_amd as mc
    from oracle import oracle as orc

    c = mc.Compiled(path=mc.graph_path("mlp_gelu"), dims={"B": batch_rows}, backend="none")
    g = c.graph()
    consts = {n["id"]: c.constant(n["id"]) for n in g["nodes"] if n["op_name"] == "const"}
    x = mc.uniform(batch_rows * 512, 1, -1.0, 1.0)
    flop = 4.0 * batch_rows * 512 * 2048

    def timed(threads: int, secs: float):
        orc.set_threads(threads)
        reps, t0 = 0, time.perf_counter()
        while True:
            orc.evaluate(g, consts, [x])
            reps += 1
            el = time.perf_counter() - t0
            if el >= secs and reps >= 2:
                break
        return el / reps, reps

    per, reps = timed(1, seconds)
    # The reference publishes one thread; all of this GPU's host share too (at
    # most 16 threads: the box's CPU share per GPU), rows split over threads.
    threads = max(1, min(os.cpu_count() or 1, 16))
    per_all, reps_all = timed(threads, seconds / 2)
    orc.set_threads(1)
    return {"value": flop / per / 1e12, "unit": "TFLOP/s", "cores": 1, "kind": "port",
            "sample": f"mlp_gelu rows 0..{batch_rows - 1} of the B=8192 batch, {reps} reps, {per * 1e3:.1f} ms/rep, "
                      f"oracle/cpu_oracle.cpp + cpu_gemm.cpp (Eigen semantics, own GEMM), 1 thread, {os.cpu_count()} host cores",
            "all_cores": {"value": flop / per_all / 1e12, "threads": threads,
                          "sample": f"the same rows, {reps_all} reps, {per_all * 1e3:.1f} ms/rep"}}


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


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # About 70 ms of timed work at B=8192; the 300 warmup steps (about 100 ms)
    # bring the GPU to its steady clock first.
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=300)
    ap.add_argument("--workload", default="mlp",
                    choices=["mlp", "gelu", "batchnorm", "gemm_fp32", "gemm_bf16", "copy"])
    ap.add_argument("--batch", type=int, default=8192)
    ap.add_argument("--quick", action="store_true", help="headline workload only (no other configs)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU; the multi-GPU sharding is a design only "
              "(see DESIGN.md). Run with --gpus 1.", file=sys.stderr)
        return 2

    import minicompiler_amd as mc

    dev = mc.device_json()
    cus = dev["cu_count"]
    log(f"device: {dev['name']} {dev['arch']} CUs={cus} clock={dev['clock_mhz']} MHz")
    line = {"metric": METRIC, "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "data": "synthetic (seeded splitmix64 uniform/normal, "
                                                            "random-init constants of the graph)"}

    if args.workload == "mlp":
        r = bench_mlp(mc, args.batch, args.steps, args.warmup)
        ks = r["kernels"]
        dom = max(ks, key=lambda e: e["ms"])
        line.update({"value": r["value"], "unit": "TFLOP/s", "ms_per_step": r["timing"]["ms_per_step"],
                     "dtype": "f32",
                     "config": {"workload": f"mlp_gelu B={args.batch} D=512 H=2048 fp32 (BASELINE config 2)",
                                "global_batch": args.batch, "matmul": ",".join(r["compiled"].matmul_kernels)}})
        unit = "TFLOP/s" if dom["bound"] == "mfma" else "GB/s"
        achieved = dom["tflops"] if dom["bound"] == "mfma" else dom["gbs"]
        line["roofline"] = {"bound": dom["bound"], "kernel": dom["launch"], "achieved": achieved,
                            "peak": dom["peak"], "unit": unit, "frac": dom["frac"], "traffic": None}
        line["kernels"] = ks
        fused = [k for k in ks if k["bound"] == "hbm"]
        line["fused_gbs"] = sum(k["bytes"] for k in fused) / (sum(k["ms"] for k in fused) * 1e-3) / 1e9 if fused else None
        line["jit_compile_ms"] = r["jit_ms"]
    else:
        line["unit"] = "GB/s" if args.workload in ("gelu", "batchnorm") else "TFLOP/s"

    if args.workload == "copy":
        # Byte-counter calibration: reads and writes 128 MiB each, known exactly.
        k = bench_elementwise_graph(mc, "copy_neg", {"M": 8192, "N": 4096}, lambda n: mc.uniform(n, 1, -1.0, 1.0),
                                    args.steps, args.warmup)
        line.update({"value": k["gbs"], "ms_per_step": k["ms_per_step"], "dtype": "f32",
                     "config": {"workload": "copy_neg (counter calibration)", **k["dims"]},
                     "roofline": {"bound": "hbm", "kernel": k["kernel"]["launch"], "achieved": k["gbs"],
                                  "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": k["frac"], "traffic": None}})
    if args.workload in ("gelu", "batchnorm") or (args.workload == "mlp" and not args.quick):
        cfgs = line.setdefault("configs", {})
        if args.workload != "batchnorm":
            cfgs["gelu_4096x4096"] = bench_elementwise_graph(
                mc, "gelu_chain", {"M": 4096, "N": 4096}, lambda n: mc.uniform(n, 1, -3.0, 3.0), args.steps, args.warmup)
            log(f"gelu: {cfgs['gelu_4096x4096']['gbs']:.0f} GB/s")
        if args.workload != "gelu":
            cfgs["batchnorm_relu_200704x256"] = bench_elementwise_graph(
                mc, "batchnorm_relu", {"R": 200704, "C": 256}, lambda n: mc.normal(n, 1, 0.0, 1.0), args.steps,
                args.warmup)
            log(f"batchnorm: {cfgs['batchnorm_relu_200704x256']['gbs']:.0f} GB/s")
        if args.workload in ("gelu", "batchnorm"):
            k = next(iter(cfgs.values()))
            line.update({"value": k["gbs"], "ms_per_step": k["ms_per_step"], "dtype": "f32",
                         "config": {"workload": k["config"], **k["dims"]},
                         "roofline": {"bound": "hbm", "kernel": k["kernel"]["launch"], "achieved": k["gbs"],
                                      "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": k["frac"], "traffic": None}})
    if args.workload == "mlp" and not args.quick:
        # BASELINE config 2's batch sweep: the small batches are timed with
        # direct launches, with hipGraph replay, and with the split count and
        # tile configuration autotuned at compile time (autotune=1).
        cfgs = line.setdefault("configs", {})
        for b in (256, 1024):
            entry = {}
            for mode, opts in (("direct", None), ("graph_replay", {"graph": 1}), ("autotuned", {"autotune": 1})):
                r = bench_mlp(mc, b, max(args.steps, 50), args.warmup, opts, WARM_SECONDS)
                entry[mode] = {"ms_per_step": r["timing"]["ms_per_step"], "tflops": r["value"],
                               "launches": r["compiled"].kernel_launches}
            cfgs[f"mlp_b{b}"] = entry
            log(f"mlp B={b}: direct {entry['direct']['ms_per_step'] * 1e3:.1f} us/step, "
                f"graph replay {entry['graph_replay']['ms_per_step'] * 1e3:.1f} us/step, "
                f"autotuned {entry['autotuned']['ms_per_step'] * 1e3:.1f} us/step")
    if args.workload == "gemm_fp32" or (args.workload == "mlp" and not args.quick):
        shapes = [(1024, 1024, 1024), (4096, 4096, 4096), (8192, 8192, 8192), (256, 256, 16384), (16, 4096, 4096)]
        g = bench_gemm_fp32(mc, cus, shapes, 10, 3)  # plus WARM_SECONDS per shape
        line.setdefault("configs", {})["gemm_fp32"] = g
        if args.workload == "gemm_fp32":
            top = g[2]
            line.update({"value": top["tflops"], "ms_per_step": top["ms"], "dtype": "f32",
                         "config": {"workload": "fp32 gemm 8192^3 (BASELINE config 4)"},
                         "roofline": {"bound": "mfma", "kernel": top["kernel"], "achieved": top["tflops"],
                                      "peak": PEAK_FP32_TFLOPS, "unit": "TFLOP/s", "frac": top["frac"], "traffic": None}})
    if args.workload == "gemm_bf16" or (args.workload == "mlp" and not args.quick):
        g = bench_gemm_lowp(mc, [(8192, 8192, 8192), (4096, 14336, 4096)], 20, 3)  # plus WARM_SECONDS
        line.setdefault("configs", {})["gemm_bf16_fp16"] = g
        line["configs"]["gemm_bf16_fp16_bias_gelu"] = bench_lowp_epilogue(
            mc, [(8192, 8192, 8192), (4096, 14336, 4096)], 20, 3)
        if args.workload == "gemm_bf16":
            top = g[0]
            line.update({"value": top["tflops"], "ms_per_step": top["ms"], "dtype": "bf16",
                         "config": {"workload": "bf16 gemm 8192^3, bf16 inputs in HBM (BASELINE config 5)"},
                         "roofline": {"bound": "mfma", "kernel": top["kernel"], "achieved": top["tflops"],
                                      "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s", "frac": top["frac"], "traffic": None}})

    if "roofline" in line:
        line["roofline"]["traffic"] = measured_traffic(line["config"]["workload"], line["roofline"]["kernel"])
    line["device"] = {k: dev[k] for k in ("name", "arch", "cu_count", "clock_mhz", "mem_clock_mhz", "bus_width_bits")}
    if not args.no_cpu_baseline and args.workload == "mlp":
        line["cpu_baseline"] = cpu_baseline(256, args.cpu_seconds)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
