"""split_k products whose K splits are added inside the GEMM launch (option
split_fold=1 in compiled graphs; off by default): the last block to finish a
split of a C tile adds the tile's partials in split order and stores C
through any fused epilogue, counting arrivals on a per-tile counter that it
leaves at zero (gemm_split_arrival.h). The order of the adds is that of the
separate sum launch (split_fold=0, and the C ABI's mc_launch_matmul), so
every output must equal that executable's bit for bit: on the narrow body
(streamed 16x64 tiles, 32x64 tiles) and on every ring configuration, with
ragged tiles, unfused and with a fused epilogue, over repeated enqueues and
graph replays; and it must lie within the reference's dot-product bound of
a float64 product (tests/test_cuda_backend.cpp:119-162)."""

import numpy as np
import pytest

from helpers import assert_close, fp32_gemm_bound, max_abs, uniform_inputs

pytestmark = pytest.mark.gpu

GEMM = "graph gemm\ninput a : f32[{m}, {k}]\ninput b : f32[{k}, {n}]\nc = matmul a, b\noutput c\n"
FOLDED = "summed in the GEMM"

# (m, k, n, options). The bench's split shapes: 16x4096x4096 (streamed
# 16x64 tiles, 4 K ranges), 256x256x16384 (32x64 tiles, 8 ranges);
# 1024x4096x2048 (the wide8 ring, 2 splits); 128x4096x4096 (64x64 tiles,
# 2 ranges); ragged M and N on 32x64 tiles; each ring
# configuration forced with a deep split, ragged where it can be.
CASES = [(16, 4096, 4096, {}), (256, 16384, 256, {}), (1024, 4096, 2048, {}), (128, 4096, 4096, {}),
         (33, 1040, 1000, {}),
         (512, 4096, 512, {"ring": "wide"}), (200, 4096, 516, {"ring": "mid"}), (32, 4096, 2048, {"ring": "thin"}),
         (300, 8192, 300, {"ring": "big"})]


def compile_pair(mc, text=None, path=None, dims=None, **opts):
    """split_k executables with and without split_fold."""
    base = {"matmul": "split_k", **opts}
    fold = mc.Compiled(text, path=path, dims=dims, options={**base, "split_fold": 1})
    plain = mc.Compiled(text, path=path, dims=dims, options=base)
    return fold, plain


@pytest.mark.parametrize("m,k,n,opts", CASES)
def test_splits_added_in_the_launch_equal_the_separate_sum(device, mc, oracle, m, k, n, opts):
    print(f"case fold gemm {m}x{k}x{n} {opts}", flush=True)
    fold, plain = compile_pair(mc, GEMM.format(m=m, k=k, n=n), **opts)
    assert FOLDED in fold.launch_names[0], fold.launch_names
    assert FOLDED not in plain.launch_names[0], plain.launch_names
    # New inputs every run: a tile that did not fold would keep the last
    # run's C. The counters are back at zero after every launch.
    for rep in range(3):
        a = oracle.uniform(m * k, 51 + 2 * rep, -1.0, 1.0)
        b = oracle.uniform(k * n, 52 + 2 * rep, -1.0, 1.0)
        want = plain.run([a, b])[0]
        got = fold.run([a, b])[0]
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"run {rep}"
    if m * n * k <= 1 << 28:
        exact, absdot = oracle.gemm_f64(a, b, m, k, n)
        g = want.astype(np.float64)
    else:
        rng = np.random.default_rng(m + n + k)
        rows, cols = rng.integers(0, m, 2000), rng.integers(0, n, 2000)
        exact, absdot = oracle.gemm_f64_sampled(a, b, rows, cols, k, n)
        g = want.astype(np.float64)[rows * n + cols]
    bad = np.abs(g - exact) > fp32_gemm_bound(exact, absdot, k)
    assert not np.any(bad), f"{np.count_nonzero(bad)} elements outside the bound"


# (graph, dims, options): the group after the GEMM runs in the last block's
# store of each tile: on streamed 16x64 tiles, on the wide ring, on the mid
# ring with ragged edges, and the MLP at a small batch (both GEMMs split).
FUSED = [("matmul_bias_relu", {"M": 16, "K": 4096, "N": 4096}, {}),
         ("matmul_bias_relu", {"M": 1024, "K": 4096, "N": 2048}, {}),
         ("matmul_bias_relu", {"M": 200, "K": 4096, "N": 516}, {"ring": "mid"}),
         ("mlp_gelu", {"B": 16}, {})]


@pytest.mark.parametrize("name,dims,opts", FUSED)
def test_fused_epilogue_in_the_folding_block_equals_the_sum_launch(device, mc, oracle, name, dims, opts):
    print(f"case fold graph {name} {dims} {opts}", flush=True)
    fold, plain = compile_pair(mc, path=mc.graph_path(name), dims=dims, **opts)
    assert any(FOLDED in s and "fused" in s for s in fold.launch_names), fold.launch_names
    assert fold.kernel_launches == plain.kernel_launches
    for rep in range(2):
        inputs = uniform_inputs(oracle, fold.input_sizes, 8 + rep)
        want = plain.run(inputs)
        got = fold.run(inputs)
        for g, w in zip(got, want):
            assert np.array_equal(g.view(np.uint32), w.view(np.uint32)), f"run {rep}"
    cpu = oracle.evaluate_compiled(fold, inputs)
    for g, c in zip(want, cpu):
        assert_close(g, c, 1e-4, 1e-4 * max(1.0, max_abs(c)), f"{name} {dims}")


def test_graph_replays_of_a_folding_launch_equal_direct_launches(device, mc, oracle):
    # Each replay starts from the counters the previous launch left at zero;
    # eager work on another executable (the separate sum) runs between the
    # replays.
    m, k, n = 16, 4096, 4096
    direct = mc.Compiled(GEMM.format(m=m, k=k, n=n), options={"matmul": "split_k"})
    replay = mc.Compiled(GEMM.format(m=m, k=k, n=n), options={"matmul": "split_k", "split_fold": 1, "graph": 1})
    assert FOLDED in replay.launch_names[0], replay.launch_names
    for rep in range(4):
        inputs = uniform_inputs(oracle, direct.input_sizes, 20 + rep)
        want = direct.run(inputs)
        replay.upload(inputs)
        replay.enqueue()  # captures at rep 0, replays afterwards
        got = replay.download()
        assert np.array_equal(got[0].view(np.uint32), want[0].view(np.uint32)), f"replay {rep}"
