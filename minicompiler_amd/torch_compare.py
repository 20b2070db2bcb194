"""The HIP backend beside PyTorch-ROCm on the same graphs, on the same stream.

    python -m minicompiler_amd.torch_compare [--quick] [--out results.json]

For each configuration (a .mcg graph and its sizes) three ways to compute the
same function run in one process, on the same seeded inputs, all on the GPU:

  minicompiler  the graph compiled by this library (all passes), its inputs
                and outputs bound to PyTorch device tensors, enqueued with
                mc_enqueue on PyTorch's current stream
  eager         PyTorch running the graph as written, op by op (the graph
                before any pass, node by node)
  idiomatic     the function as a PyTorch user writes it, with its fused
                library ops (F.gelu(approximate="tanh"), torch.addmm,
                F.batch_norm)

Each call is timed with torch.cuda events recorded on the shared stream from
before the call to after its last kernel, so host launch overhead counts
whenever the GPU waits for it. After a warm-up measured in time (the GPU
raises its clock only under sustained load), the variants run in rounds of
one call each, in a freshly shuffled (seeded) order per round; the result is
each variant's median and the median over rounds of PyTorch time /
minicompiler time. Every variant's outputs are checked against
minicompiler's (max |difference| / max(1, max |minicompiler|) <= 1e-4).
FP32 matmuls are full FP32 everywhere (TF32 off in PyTorch).

This is the GPU path of the reference's bench/torch_compare.py (its caller
of bench/capi.cpp); torch.compile is left out (its GPU code generator is not
part of this build's toolchain)."""

from __future__ import annotations

import argparse
import json
import random
import statistics
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

import minicompiler_amd as mc  # noqa: E402

# (graph, dims, input distribution (kind, a, b) per input, label)
CONFIGS = [
    ("gelu_chain", {"M": 256, "N": 4096}, [("uniform", -3.0, 3.0)], "GELU 256x4096 (4 MB)"),
    ("gelu_chain", {"M": 4096, "N": 4096}, [("uniform", -3.0, 3.0)], "GELU 4096x4096 (64 MB)"),
    ("batchnorm_relu", {"R": 200704, "C": 256}, [("normal", 0.0, 1.0)], "BatchNorm+ReLU 200704x256"),
    ("matmul_bias_relu", {"M": 2048, "K": 1024, "N": 1024}, [("uniform", -1.0, 1.0)], "2048x1024 @ 1024x1024 + bias, ReLU"),
    ("mlp_gelu", {"B": 256}, [("uniform", -1.0, 1.0)], "MLP B=256"),
    ("mlp_gelu", {"B": 1024}, [("uniform", -1.0, 1.0)], "MLP B=1024"),
    ("mlp_gelu", {"B": 8192}, [("uniform", -1.0, 1.0)], "MLP B=8192"),
]
QUICK = [CONFIGS[1], CONFIGS[4], CONFIGS[6]]

UNARY = {"neg": "neg", "exp": "exp", "log": "log", "sqrt": "sqrt", "relu": "relu", "sigmoid": "sigmoid",
         "tanh": "tanh"}
BINARY = {"add": "add", "sub": "sub", "mul": "mul", "div": "div"}


def make_inputs(sizes, dists, seed: int = 1) -> list[np.ndarray]:
    """Input k from seed + k, as mcc makes them."""
    out = []
    for k, n in enumerate(sizes):
        kind, a, b = dists[k]
        out.append(mc.uniform(int(n), seed + k, a, b) if kind == "uniform" else mc.normal(int(n), seed + k, a, b))
    return out


def graph_constants(compiled) -> tuple[dict, dict[int, np.ndarray]]:
    g = compiled.graph()
    return g, {n["id"]: compiled.constant(n["id"]) for n in g["nodes"] if n["op_name"] == "const"}


def eager_function(graph: dict, constants: dict, torch, device):
    """The graph as written, one PyTorch op per node (numpy-style
    broadcasting, as the graph's binary ops broadcast). Returns f(*inputs)
    -> tuple of outputs."""
    nodes = graph["nodes"]
    consts = {i: torch.from_numpy(np.ascontiguousarray(v)).to(device).reshape(nodes[i]["shape"])
              for i, v in constants.items()}

    def run(*inputs):
        values = dict(consts)
        for k, nid in enumerate(graph["inputs"]):
            values[nid] = inputs[k]
        for node in nodes:
            nid, op = node["id"], node["op_name"]
            if op in ("input", "const"):
                continue
            args = [values[i] for i in node["inputs"]]
            if op == "matmul":
                values[nid] = torch.matmul(args[0], args[1])
            elif op in UNARY:
                values[nid] = getattr(torch, UNARY[op])(args[0])
            elif op in BINARY:
                values[nid] = getattr(torch, BINARY[op])(args[0], args[1])
            else:
                raise ValueError(f"no PyTorch op for graph op '{op}'")
        return tuple(values[o] for o in graph["outputs"])

    return run


def idiomatic_function(name: str, graph: dict, constants: dict, torch, device):
    """The same function with PyTorch's fused library ops."""
    import torch.nn.functional as F

    by_name = {n["name"]: torch.from_numpy(np.ascontiguousarray(constants[n["id"]])).to(device).reshape(n["shape"])
               for n in graph["nodes"] if n["op_name"] == "const"}
    if name == "gelu_chain":
        return lambda x: (F.gelu(x, approximate="tanh"),)
    if name == "matmul_bias_relu":
        w, b = by_name["w"], by_name["b"]
        return lambda x: (torch.relu(torch.addmm(b, x, w)),)
    if name == "matmul_bias_gelu":
        w, b = by_name["w"], by_name["bias"]
        return lambda x: (F.gelu(torch.addmm(b, x, w), approximate="tanh"),)
    if name == "mlp_gelu":
        c = by_name
        return lambda x: (torch.addmm(c["b2"], F.gelu(torch.addmm(c["b1"], x, c["w1"]), approximate="tanh"),
                                      c["w2"]) + x,)
    if name == "batchnorm_relu":
        c = by_name
        eps = float(c["eps"].reshape(-1)[0].item())
        return lambda x: (torch.relu(F.batch_norm(x, c["mean"], c["var"], c["gamma"], c["beta"], training=False,
                                                  eps=eps)),)
    raise ValueError(name)


def worst_difference(actual, expected) -> float:
    worst = 0.0
    for a, e in zip(actual, expected):
        a = np.asarray(a, dtype=np.float64).ravel()
        e = np.asarray(e, dtype=np.float64).ravel()
        worst = max(worst, float(np.max(np.abs(a - e)) / max(1.0, float(np.max(np.abs(e))))))
    return worst


def time_rounds(fns: dict, torch, warm_seconds: float, seconds: float, seed: int = 20261201) -> dict:
    """Per-call times (ms) of each function, in shuffled interleaved rounds
    after a warm-up of `warm_seconds`."""
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def timed(fn) -> float:
        start.record()
        fn()
        stop.record()
        stop.synchronize()
        return start.elapsed_time(stop)

    names = list(fns)
    until = time.perf_counter() + warm_seconds
    while time.perf_counter() < until:
        for n in names:
            timed(fns[n])
    probe = sum(statistics.median(timed(fns[n]) for _ in range(3)) for n in names)
    rounds = max(20, min(2000, int(seconds * 1000.0 / max(probe, 1e-3))))
    samples = {n: [] for n in names}
    rng = random.Random(seed)
    order = list(names)
    for _ in range(rounds):
        rng.shuffle(order)
        for n in order:
            samples[n].append(timed(fns[n]))
    return samples


def compare(name: str, dims: dict, dists, label: str, torch, warm_seconds: float, seconds: float) -> dict:
    device = torch.device("cuda")
    ours = mc.Compiled(path=mc.graph_path(name), dims=dims)
    raw = mc.Compiled(path=mc.graph_path(name), dims=dims, passes="none", backend="none")
    graph, constants = graph_constants(raw)
    host_inputs = make_inputs(ours.input_sizes, dists)
    x = [torch.from_numpy(a).to(device).reshape(graph["nodes"][nid]["shape"])
         for a, nid in zip(host_inputs, graph["inputs"])]
    outs = [torch.empty(graph["nodes"][o]["shape"], dtype=torch.float32, device=device) for o in graph["outputs"]]
    ours.bind_inputs([t.data_ptr() for t in x])
    ours.bind_outputs([t.data_ptr() for t in outs])
    stream = torch.cuda.current_stream().cuda_stream
    if not stream:
        # 0 would mean the executable's own stream, not PyTorch's.
        raise ValueError("run under a non-default PyTorch stream (torch.cuda.stream(torch.cuda.Stream()))")

    def run_ours():
        ours.enqueue(stream)

    eager = eager_function(graph, constants, torch, device)
    idiom = idiomatic_function(name, graph, constants, torch, device)
    fns = {"minicompiler": run_ours, "eager": lambda: eager(*x), "idiomatic": lambda: idiom(*x)}

    run_ours()
    torch.cuda.synchronize()
    reference = [o.cpu().numpy() for o in outs]
    check = {n: worst_difference([t.cpu().numpy() for t in f(*x)], reference)
             for n, f in (("eager", eager), ("idiomatic", idiom))}
    samples = time_rounds(fns, torch, warm_seconds, seconds)
    med = {n: statistics.median(v) for n, v in samples.items()}
    ratios = {n: statistics.median(samples[n][i] / samples["minicompiler"][i] for i in range(len(samples[n])))
              for n in ("eager", "idiomatic")}
    result = {"graph": name, "dims": dims, "label": label, "rounds": len(samples["minicompiler"]),
              "median_ms": med, "torch_over_minicompiler": ratios, "max_normwise_difference": check,
              "minicompiler_launches": ours.kernel_launches, "matmul_kernels": list(ours.matmul_kernels)}
    ok = all(v <= 1e-4 for v in check.values())
    result["outputs_agree"] = ok
    print(f"{label}: minicompiler {med['minicompiler'] * 1e3:.1f} us, eager {med['eager'] * 1e3:.1f} us "
          f"(x{ratios['eager']:.2f}), idiomatic {med['idiomatic'] * 1e3:.1f} us (x{ratios['idiomatic']:.2f}); "
          f"outputs {'agree' if ok else 'DIFFER'} ({max(check.values()):.1e})", file=sys.stderr, flush=True)
    ours.close()
    return result


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--quick", action="store_true", help="GELU 4096^2 and the MLP at B=256 and 8192 only")
    ap.add_argument("--warmup-seconds", type=float, default=0.5)
    ap.add_argument("--seconds", type=float, default=1.0, help="timed seconds per configuration")
    ap.add_argument("--out", help="also write the JSON here")
    args = ap.parse_args(argv)

    import torch

    if not torch.cuda.is_available():
        print("torch_compare: no GPU visible to PyTorch", file=sys.stderr)
        return 2
    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.allow_tf32 = False
    # One stream for every variant (default priority); PyTorch's legacy
    # default stream has no handle to pass to mc_enqueue.
    with torch.cuda.stream(torch.cuda.Stream()):
        results = [compare(n, d, dist, label, torch, args.warmup_seconds, args.seconds)
                   for n, d, dist, label in (QUICK if args.quick else CONFIGS)]
    doc = {"torch": torch.__version__, "device": torch.cuda.get_device_name(0), "configs": results}
    text = json.dumps(doc)
    if args.out:
        Path(args.out).write_text(text + "\n")
    print(text)
    return 0 if all(r["outputs_agree"] for r in results) else 1


if __name__ == "__main__":
    sys.exit(main())
