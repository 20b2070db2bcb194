"""The narrow-tile FP32 body (gemm_f32_narrow.h: 16x32, 16x64, 32x64 or 64x64
tiles on 16x16x4 MFMAs, K cut over waves and over ranges of the grid), through the C
ABI and in compiled graphs.

It serves split_k products whose tiles number at most one per CU, so its
results are checked against float64 dot products within the reference's
dot-product bound (tests/test_cuda_backend.cpp:119-162), with a NaN guard
past the end of C; it is deterministic (a fixed order of adds); and a
fused epilogue on it gives the bits of the unfused graph."""

import numpy as np
import pytest

from helpers import assert_close, fp32_gemm_bound, max_abs, uniform_inputs

pytestmark = pytest.mark.gpu

GUARD = 4096

# (m, k, n, splits): one row, M < 16, exactly 16, ragged M past a 32-row
# tile, N not a multiple of 64 (and not of 8), K not a multiple of the
# split, a split count above what the plan would take, the bench shapes.
# The short-K tile shapes too: 256x2048x512 and 300x96x260 on 16x32 tiles,
# 512^3 and 200x512x640 (ragged M) on 16x64 tiles, unsplit. Waves with 32
# groups of K or more load two groups per batch (256x2048x512 on 16x32
# tiles, 256x256x16384 in 8 ranges), and 64x2064x260 gives them 33 (an odd
# count: a last group on its own). 64x64 tiles: 1024^3 unsplit, 1000x528x1000
# unsplit with ragged edges, 128x4096x4096 and 300x4112x1000 (ragged) in 2
# K ranges.
SHAPES = [(1, 16, 4, 1), (5, 96, 260, 3), (16, 4096, 4096, 8), (33, 1040, 1000, 4), (300, 96, 260, 2),
          (256, 512, 2048, 8), (256, 2048, 512, 32), (512, 512, 512, 8), (16, 64, 68, 64), (256, 16384, 256, 64),
          (200, 512, 640, 4), (64, 2064, 260, 1), (1024, 1024, 1024, 4), (1000, 528, 1000, 4), (128, 4096, 4096, 8),
          (300, 4112, 1000, 4)]


def run(mc, ring, a, b, m, k, n, splits):
    da, db = mc.DeviceBuffer.from_array(a), mc.DeviceBuffer.from_array(b)
    ws = mc.DeviceBuffer(mc.matmul_workspace_bytes("split_k", m, n, splits)) if splits > 1 else None
    dc = mc.DeviceBuffer.from_array(np.full(m * n + GUARD, np.nan, dtype=np.float32))
    mc.launch_matmul_cfg("split_k", da.ptr, db.ptr, dc.ptr, m, n, k, None, splits, ws.ptr if ws else None, ring)
    mc.synchronize()
    out = dc.download()
    assert np.all(np.isnan(out[m * n:])), "a write past the end of C"
    assert not np.any(np.isnan(out[:m * n])), "an element of C was not written"
    return out[:m * n]


@pytest.mark.parametrize("m,k,n,splits", SHAPES)
def test_narrow_split_k_is_within_the_dot_product_bound_and_deterministic(device, mc, oracle, m, k, n, splits):
    print(f"case narrow {m}x{k}x{n} splits={splits}", flush=True)
    a = oracle.uniform(m * k, 31, -1.0, 1.0)
    b = oracle.uniform(k * n, 32, -1.0, 1.0)
    got = run(mc, "narrow", a, b, m, k, n, splits)
    again = run(mc, "narrow", a, b, m, k, n, splits)
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))
    if m * n * k <= 1 << 28:
        exact, absdot = oracle.gemm_f64(a, b, m, k, n)
        g = got.astype(np.float64)
    else:
        rng = np.random.default_rng(m + n + k)
        rows, cols = rng.integers(0, m, 2000), rng.integers(0, n, 2000)
        exact, absdot = oracle.gemm_f64_sampled(a, b, rows, cols, k, n)
        g = got.astype(np.float64)[rows * n + cols]
    bad = np.abs(g - exact) > fp32_gemm_bound(exact, absdot, k)
    assert not np.any(bad), f"{np.count_nonzero(bad)} elements outside the bound"


def test_the_plan_takes_narrow_tiles_only_where_they_fit(device, mc, oracle):
    # 256x2048x512 (256 tiles of 32x64), 16x4096x4096 (64 of 16x64) and
    # 1024x1024x1024 (256 of 64x64) run narrow; 1024x4096x2048 (K past 2048,
    # 512 tiles of 64x64) keeps the ring, in 2 splits. The plan's split_k launch then equals the forced
    # narrow launch (same plan) bit for bit, or the forced wide8 ring's.
    for (m, k, n), body in (((256, 512, 2048), "narrow"), ((16, 4096, 4096), "narrow"),
                            ((1024, 1024, 1024), "narrow"), ((1024, 4096, 2048), "wide8")):
        print(f"case plan {m}x{k}x{n} -> {body}", flush=True)
        a = oracle.uniform(m * k, 41, -1.0, 1.0)
        b = oracle.uniform(k * n, 42, -1.0, 1.0)
        splits = mc.matmul_splits("split_k", m, n, k, int(device["cu_count"]))
        planned = run(mc, "auto", a, b, m, k, n, splits)
        forced = run(mc, body, a, b, m, k, n, splits)
        assert np.array_equal(planned.view(np.uint32), forced.view(np.uint32)), (m, k, n)


def test_a_forced_narrow_launch_the_product_cannot_take_is_an_error(device, mc):
    da, db, dc = mc.DeviceBuffer(4 * 64 * 40), mc.DeviceBuffer(4 * 40 * 64), mc.DeviceBuffer(4 * 64 * 64)
    with pytest.raises(mc.HipError):  # K not a multiple of 16
        mc.launch_matmul_cfg("split_k", da.ptr, db.ptr, dc.ptr, 64, 64, 40, None, 1, None, "narrow")
    with pytest.raises(mc.HipError):  # split_k only
        mc.launch_matmul_cfg("double_buffered", da.ptr, db.ptr, dc.ptr, 64, 64, 32, None, 1, None, "narrow")


GRAPHS = [("mlp_gelu", {"B": 256}), ("mlp_gelu", {"B": 16}), ("matmul_bias_relu", {"M": 16, "K": 1024, "N": 1000}),
          ("matmul_bias_relu", {"M": 96, "K": 512, "N": 512}), ("matmul_bias_relu", {"M": 512, "K": 512, "N": 512}),
          ("matmul_bias_relu", {"M": 1024, "K": 1024, "N": 1024})]


@pytest.mark.parametrize("name,dims", GRAPHS)
def test_graphs_on_narrow_tiles_fuse_their_groups_bit_for_bit_and_match_the_oracle(device, mc, oracle, name, dims):
    # split_k (auto at these sizes) plans the narrow body; the group after
    # each GEMM runs in its store (one K range) or in the split sum.
    print(f"case narrow graph {name} {dims}", flush=True)
    opts = {"matmul": "split_k"}
    fused = mc.Compiled(path=mc.graph_path(name), dims=dims, options=opts)
    plain = mc.Compiled(path=mc.graph_path(name), dims=dims, options={**opts, "epilogue": 0})
    sources = "\n".join(fused.kernel_sources)
    assert "mc_gemm_f32_narrow<" in sources, fused.launch_names
    assert any(len(ids) > 1 for ids in fused.launch_nodes)
    inputs = uniform_inputs(oracle, fused.input_sizes, 7)
    x, y = fused.run(inputs), plain.run(inputs)
    for p, q in zip(x, y):
        assert np.array_equal(p.view(np.uint32), q.view(np.uint32))
    cpu = oracle.evaluate_compiled(fused, inputs)
    for p, c in zip(x, cpu):
        assert_close(p, c, 1e-4, 1e-4 * max(1.0, max_abs(c)), f"{name} {dims}")


def test_short_k_products_run_on_the_tile_shape_that_gives_most_cus_a_tile(device, mc):
    # On 256 CUs: the MLP at B=256 runs GEMM1 (256x2048x512) on 32x64 tiles
    # and GEMM2 (256x512x2048) on 16x32 tiles, 512^3 on 16x64 tiles, 1024^3
    # on 64x64 tiles.
    if int(device["cu_count"]) != 256:
        pytest.skip("tile counts are for 256 CUs")
    opts = {"matmul": "split_k"}
    mlp = "\n".join(mc.Compiled(path=mc.graph_path("mlp_gelu"), dims={"B": 256}, options=opts).kernel_sources)
    assert "mc_gemm_f32_narrow<McNarrow32>" in mlp and "mc_gemm_f32_narrow<McNarrow16x32>" in mlp
    sq = "\n".join(mc.Compiled(path=mc.graph_path("matmul_bias_relu"), dims={"M": 512, "K": 512, "N": 512},
                               options=opts).kernel_sources)
    assert "mc_gemm_f32_narrow<McNarrow16x64>" in sq
    big = "\n".join(mc.Compiled(path=mc.graph_path("matmul_bias_relu"), dims={"M": 1024, "K": 1024, "N": 1024},
                                options=opts).kernel_sources)
    assert "mc_gemm_f32_narrow<McNarrow64>" in big
    # The MLP at B=1024: GEMM1 (1024x2048x512) on 64x64 tiles, two per CU.
    mlp = "\n".join(mc.Compiled(path=mc.graph_path("mlp_gelu"), dims={"B": 1024}, options=opts).kernel_sources)
    assert "mc_gemm_f32_narrow<McNarrow64>" in mlp


@pytest.mark.parametrize("m,k,n,splits,ranges", [(256, 16384, 256, 64, 8), (16, 4096, 4096, 8, 4),
                                                 (1024, 1024, 1024, 4, 1), (2048, 2048, 2048, 1, 1)])
def test_the_k_ranges_that_run_are_reported(device, mc, m, k, n, splits, ranges):
    # The split count is an upper bound for the narrow-tile body: the query,
    # the compiled graph's launch name and the plan agree on what runs.
    print(f"case k ranges {m}x{k}x{n} splits={splits}", flush=True)
    kernel = "split_k" if splits > 1 else "double_buffered"
    assert mc.matmul_k_ranges(kernel, m, n, k, splits) == ranges
    c = mc.Compiled(f"graph g\ninput a : f32[{m}, {k}]\ninput b : f32[{k}, {n}]\nc = matmul a, b\noutput c\n",
                    options={"matmul": kernel, "split_fold": 0})
    (name,) = [nm for nm in c.launch_names if nm.startswith("matmul")]
    if splits == 1:
        assert "splits=" not in name, name
    elif ranges == splits:
        assert f"splits={ranges}" in name and " of " not in name, name
    else:
        assert f"splits={ranges} of {splits}" in name, name
