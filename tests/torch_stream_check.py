"""Child process of tests/test_gpu_torch.py: compiled graphs bound to
PyTorch tensors and enqueued on PyTorch's stream, checked against the CPU
oracle and PyTorch's library ops. PyTorch is imported and its GPU context
made before the library loads: PyTorch ships its own HIP runtime under the
same soname, and the first one loaded serves both. Prints one JSON line per
case and exits 1 if any case fails."""

import json
import sys
import traceback
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))

# (graph, dims, input distributions, tolerance against the oracle: rtol and
# that fraction of the scale; 1e-5 for elementwise graphs, 1e-4 with FP32
# GEMMs).
CASES = [("gelu_chain", {"M": 256, "N": 4096}, [("uniform", -3.0, 3.0)], 1e-5),
         ("batchnorm_relu", {"R": 512, "C": 256}, [("normal", 0.0, 1.0)], 1e-5),
         ("mlp_gelu", {"B": 256}, [("uniform", -1.0, 1.0)], 1e-4),
         ("matmul_bias_gelu", {"M": 512, "K": 1024, "N": 768}, [("uniform", -1.0, 1.0)], 1e-4)]


def check(mc, oracle, tc, helpers, name, dims, dists, tol) -> dict:
    ours = mc.Compiled(path=mc.graph_path(name), dims=dims)
    raw = mc.Compiled(path=mc.graph_path(name), dims=dims, passes="none", backend="none")
    graph, constants = tc.graph_constants(raw)
    host = tc.make_inputs(ours.input_sizes, dists)
    cuda = torch.device("cuda")
    with torch.cuda.stream(torch.cuda.Stream()):
        stream = torch.cuda.current_stream()
        x = [torch.from_numpy(a).to(cuda).reshape(graph["nodes"][nid]["shape"])
             for a, nid in zip(host, graph["inputs"])]
        outs = [torch.full(graph["nodes"][o]["shape"], float("nan"), dtype=torch.float32, device=cuda)
                for o in graph["outputs"]]
        ours.bind_inputs([t.data_ptr() for t in x])
        ours.bind_outputs([t.data_ptr() for t in outs])
        # PyTorch writes the input just before the launches, on the same
        # stream, and reads the outputs just after them.
        x[0].mul_(-1.0)
        ours.enqueue(stream.cuda_stream)
        after = [o.clone() for o in outs]
        stream.synchronize()
        got = [t.cpu().numpy().reshape(-1) for t in after]
        idiom = tc.idiomatic_function(name, graph, constants, torch, cuda)
        theirs = [t.cpu().numpy().reshape(-1) for t in idiom(*x)]
    ours.close()
    want = oracle.evaluate(graph, constants, [-host[0]] + host[1:])
    for g, w in zip(got, want):
        if np.any(np.isnan(g)):
            raise AssertionError("an output element was not written before PyTorch read it")
        helpers.assert_close(g, w, tol, tol * max(1.0, helpers.max_abs(w)), f"{name} against the oracle")
    diff = tc.worst_difference(theirs, got)
    if diff > 1e-4:
        raise AssertionError(f"{name}: PyTorch's library ops differ by {diff:.2e}")
    return {"graph": name, "dims": dims, "launches": len(got), "pytorch_difference": diff}


def main() -> int:
    if not torch.cuda.is_available():
        print(json.dumps({"error": "PyTorch sees no GPU"}), flush=True)
        return 1
    torch.zeros(1, device="cuda")  # PyTorch's GPU context first
    import helpers
    import minicompiler_amd as mc
    from minicompiler_amd import torch_compare as tc
    from oracle import oracle

    mc.library()
    failed = 0
    for name, dims, dists, tol in CASES:
        print(f"case torch {name} {dims}", file=sys.stderr, flush=True)
        try:
            print(json.dumps({"ok": True, **check(mc, oracle, tc, helpers, name, dims, dists, tol)}), flush=True)
        except Exception:
            failed += 1
            print(json.dumps({"ok": False, "graph": name, "error": traceback.format_exc()}), flush=True)
    return 1 if failed else 0


if __name__ == "__main__":
    sys.exit(main())
