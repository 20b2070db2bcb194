"""The PyTorch side of minicompiler_amd.torch_compare, checked on the CPU
against the oracle: the graph translated op by op (eager) and the
library-op version (idiomatic) compute the graph's function within the
fused-fp32 / FP32-GEMM tolerance (the GPU side-by-side then checks every
variant against minicompiler's outputs the same way)."""

import numpy as np
import pytest

from helpers import assert_close, max_abs

torch = pytest.importorskip("torch")

CASES = [("gelu_chain", {"M": 8, "N": 96}, [("uniform", -3.0, 3.0)]),
         ("batchnorm_relu", {"R": 50, "C": 16}, [("normal", 0.0, 1.0)]),
         ("matmul_bias_relu", {"M": 12, "K": 40, "N": 24}, [("uniform", -1.0, 1.0)]),
         ("matmul_bias_gelu", {"M": 10, "K": 64, "N": 20}, [("uniform", -1.0, 1.0)]),
         ("mlp_gelu", {"B": 6}, [("uniform", -1.0, 1.0)])]


@pytest.mark.parametrize("name,dims,dists", CASES)
def test_eager_and_idiomatic_torch_match_the_oracle(mc, oracle, name, dims, dists):
    from minicompiler_amd import torch_compare as tc

    raw = mc.Compiled(path=mc.graph_path(name), dims=dims, passes="none", backend="none")
    graph, constants = tc.graph_constants(raw)
    inputs = tc.make_inputs(raw.input_sizes, dists)
    want = oracle.evaluate(graph, constants, inputs)[0]
    dev = torch.device("cpu")
    x = [torch.from_numpy(a).reshape(graph["nodes"][nid]["shape"]) for a, nid in zip(inputs, graph["inputs"])]
    tol = 1e-4 if any(n["op_name"] == "matmul" for n in graph["nodes"]) else 1e-5
    for fn in (tc.eager_function(graph, constants, torch, dev), tc.idiomatic_function(name, graph, constants, torch, dev)):
        got = fn(*x)[0].numpy().reshape(-1)
        assert_close(got, want, tol, tol * max(1.0, max_abs(want)), name)
    assert tc.worst_difference([want], [want]) == 0.0
