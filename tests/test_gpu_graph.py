"""hipGraph replay of enqueue (option graph=1): the first enqueue captures
the executable's launches into a graph, later ones replay it. Each replay,
with eager uploads and synchronisations between replays, must equal an
executable that launches directly, bit for bit, and the CPU oracle within
the graph's tolerance (rtol 1e-5 plus 1e-5 of the scale for elementwise
graphs, 1e-4 with FP32 GEMMs, the tensor-core bound's scale for bf16);
binding other buffers captures a graph for that binding, kept beside
the others so that buffer sets can rotate. (The reference runs graphs only
around its GEMM timing, bench/bench_cuda.cpp:445-493; replaying a whole
enqueue is this build's.)"""

import numpy as np
import pytest

from helpers import assert_close, max_abs, uniform_inputs

pytestmark = pytest.mark.gpu

# (graph, dims, options, rtol against the oracle). The bf16 MLP's inputs
# are rounded to bf16 (u = 2^-8) before K = 512 and 2048 products: 1e-2 of
# the scale covers the sqrt(K) u growth of BASELINE's bound.
CASES = [("mlp_gelu", {"B": 256}, {}, 1e-4), ("mlp_gelu", {"B": 256}, {"matmul": "tensor_core_bf16"}, 1e-2),
         ("gelu_chain", {"M": 64, "N": 4096}, {}, 1e-5), ("batchnorm_relu", {"R": 512, "C": 256}, {}, 1e-5)]


@pytest.mark.parametrize("name,dims,opts,rtol", CASES[:3])
def test_runs_of_captured_steps_equal_direct_launches(device, mc, oracle, name, dims, opts, rtol):
    # enqueue_steps on one set of buffers under graph replay: 37 steps are
    # two replays of a 16-step graph and five of the one-step graph. New
    # inputs before each call; eager work between the calls.
    print(f"case graph steps {name} {dims} {opts}", flush=True)
    direct = mc.Compiled(path=mc.graph_path(name), dims=dims, options=opts)
    replay = mc.Compiled(path=mc.graph_path(name), dims=dims, options={**opts, "graph": 1})
    for rep, steps in enumerate((37, 16, 3)):
        inputs = uniform_inputs(oracle, direct.input_sizes, 40 + rep)
        want = direct.run(inputs)
        replay.upload(inputs)
        replay.enqueue_steps(steps)
        got = replay.download()
        for g, w in zip(got, want):
            assert np.array_equal(g.view(np.uint32), w.view(np.uint32)), f"call {rep} ({steps} steps)"
    cpu = oracle.evaluate_compiled(direct, inputs)
    for g, c in zip(got, cpu):
        assert_close(g, c, rtol, rtol * max(1.0, max_abs(c)), "against the oracle")


@pytest.mark.parametrize("name,dims,opts,rtol", CASES)
def test_every_graph_replay_equals_direct_launches(device, mc, oracle, name, dims, opts, rtol):
    print(f"case graph {name} {dims} {opts}", flush=True)
    direct = mc.Compiled(path=mc.graph_path(name), dims=dims, options=opts)
    replay = mc.Compiled(path=mc.graph_path(name), dims=dims, options={**opts, "graph": 1})
    want = None
    for rep in range(4):
        inputs = uniform_inputs(oracle, direct.input_sizes, 10 + rep)
        want = direct.run(inputs)  # eager work between the replays
        replay.upload(inputs)
        replay.enqueue()  # captures at rep 0, replays afterwards
        got = replay.download()
        for g, w in zip(got, want):
            assert np.array_equal(g.view(np.uint32), w.view(np.uint32)), f"replay {rep}"
        cpu = oracle.evaluate_compiled(direct, inputs)
        for g, c in zip(got, cpu):
            assert_close(g, c, rtol, rtol * max(1.0, max_abs(c)), f"replay {rep} against the oracle")
    # Binding an output buffer captures again; the replay writes it in place.
    out = mc.DeviceBuffer(4 * replay.output_sizes[0])
    out.fill_bytes(0xFF)
    replay.bind_outputs([out.ptr] + [None] * (len(replay.output_sizes) - 1))
    for _ in range(2):
        replay.enqueue()
        replay.synchronize()
        assert np.array_equal(out.download().view(np.uint32), want[0].view(np.uint32))


@pytest.mark.parametrize("name,dims,opts,rtol", CASES[:2])
def test_replay_over_rotating_buffer_sets_equals_direct_launches(device, mc, oracle, name, dims, opts, rtol):
    # graph=1 with enqueue_steps over two buffer sets: each step binds its
    # set, so a graph is captured per set and replayed when the set comes
    # round again; rebinding never destroys a graph that may still run.
    # Every set's output, after 2, 5 and 1 steps, must equal direct launches
    # on that set's inputs, bit for bit.
    print(f"case graph sets {name} {dims} {opts}", flush=True)
    direct = mc.Compiled(path=mc.graph_path(name), dims=dims, options=opts)
    replay = mc.Compiled(path=mc.graph_path(name), dims=dims, options={**opts, "graph": 1})
    inputs = [uniform_inputs(oracle, direct.input_sizes, 60 + s) for s in range(2)]
    want = [direct.run(x) for x in inputs]
    bufs = []
    for x in inputs:
        ins = [mc.DeviceBuffer.from_array(a) for a in x]
        outs = [mc.DeviceBuffer(4 * n) for n in replay.output_sizes]
        bufs.append((ins, outs))
    sets = [([b.ptr for b in ins], [b.ptr for b in outs]) for ins, outs in bufs]
    for steps in (2, 5, 1):
        for _, outs in bufs:
            for b in outs:
                b.fill_bytes(0xFF)
        replay.enqueue_steps(steps, sets=sets)
        replay.synchronize()
        for s in range(min(steps, 2)):
            got = [b.download() for b in bufs[s][1]]
            for g, w in zip(got, want[s]):
                assert np.array_equal(g.view(np.uint32), w.view(np.uint32)), f"set {s} after {steps} steps"
    cpu = oracle.evaluate_compiled(direct, inputs[0])
    got = [b.download() for b in bufs[0][1]]
    for g, c in zip(got, cpu):
        assert_close(g, c, rtol, rtol * max(1.0, max_abs(c)), "against the oracle")
