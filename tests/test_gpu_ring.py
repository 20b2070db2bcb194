"""The FP32 ring body against the two-stage body, through the C ABI.

double_buffered and split_k run the ring body (gemm_f32_ring.h) when K is a
multiple of 32 and N of 4; vectorized always runs the two-stage body
(gemm_f32_mfma.h, one stage). Both accumulate every C element by the same
v_mfma_f32_32x32x2_f32 sequence, so the outputs must be identical bit for
bit, and within the reference's dot-product bound
(tests/test_cuda_backend.cpp:119-162). The shapes reach the ring
configurations the planner picks on a 256-CU MI355X (128x128 tiles with the
fetch staged through registers, in two 4-wave blocks or one 8-wave block per
CU; 32x128 tiles for M <= 32), blocks that take several tiles, odd and even
K-step counts, ragged edges and a grid that is not a multiple of 8; the fused
test also forces the 256x256 tiles."""

import numpy as np
import pytest

from helpers import assert_close, fp32_gemm_bound, max_abs, uniform_inputs

pytestmark = pytest.mark.gpu

GUARD = 4096  # floats after C, prefilled with NaN; must stay untouched

# (m, k, n) and the configuration the plan picks on 256 CUs: 128x128 tiles in
# two blocks per CU, ragged M and N, two tiles per block (1024 tiles); one K
# step per tile and four tiles per block (2048 tiles: every other tile starts
# the staged loop on an odd step); ragged, one tile per block (512 tiles);
# three K steps (a pair of steps, then one) with some CUs holding one block
# (304 tiles); one 8-wave block per CU with a grid of 9 (not a multiple of 8)
# and with 256 tiles (the class of the MLP's second GEMM); one row, one K
# step; M <= 32 (32x128 tiles, 6 stages), N ragged and a grid of 33; two
# tiles. (256x256 tiles run only when forced: the fused test below.)
SHAPES = [(4000, 64, 4000), (4096, 32, 8192), (4000, 64, 2000), (2048, 96, 2432), (300, 96, 260), (8192, 256, 512),
          (1, 32, 4), (16, 1024, 4100), (32, 64, 256)]


def run(mc, kernel, da, db, m, n, k):
    dc = mc.DeviceBuffer.from_array(np.full(m * n + GUARD, np.nan, dtype=np.float32))
    mc.launch_matmul(kernel, da.ptr, db.ptr, dc.ptr, m, n, k)
    mc.synchronize()
    out = dc.download()
    assert np.all(np.isnan(out[m * n:])), f"{kernel}: a write past the end of C"
    assert not np.any(np.isnan(out[:m * n])), f"{kernel}: an element of C was not written"
    return out[:m * n]


@pytest.mark.parametrize("m,k,n", SHAPES)
def test_ring_body_equals_the_two_stage_body_bit_for_bit(device, mc, oracle, m, k, n):
    print(f"case ring {m}x{k}x{n}", flush=True)
    a = oracle.uniform(m * k, 11, -1.0, 1.0)
    b = oracle.uniform(k * n, 12, -1.0, 1.0)
    da, db = mc.DeviceBuffer.from_array(a), mc.DeviceBuffer.from_array(b)
    two = run(mc, "vectorized", da, db, m, n, k)
    ring = run(mc, "double_buffered", da, db, m, n, k)
    assert np.array_equal(two.view(np.uint32), ring.view(np.uint32))
    exact, absdot = oracle.gemm_f64(a, b, m, k, n)
    bound = fp32_gemm_bound(exact, absdot, k)
    assert np.all(np.abs(ring.astype(np.float64) - exact) <= bound)


@pytest.mark.parametrize("batch,ring,config", [(4096, None, "McRingWide"), (8192, None, "McRingWide"),
                                               (8192, "big", "McRingBig")])
def test_fused_epilogue_on_the_ring_equals_the_two_stage_body(device, mc, oracle, batch, ring, config):
    # The MLP block: GEMM1 (B x 2048 x 512) runs the ring (128x128 tiles in
    # two blocks per CU, as the planner picks, or 256x256 tiles when forced)
    # with bias+GELU fused into its store; GEMM2 (B x 512 x 2048) the 128x128
    # ring with one block per CU, with b2 + residual (a fused GEMM keeps the
    # 4-wave blocks where an unfused one would take the 8-wave block). The
    # vectorized graph runs the two-stage body (also fused): identical bits
    # throughout.
    print(f"case mlp B={batch} ring={ring}", flush=True)
    dims = {"B": batch}
    options = {"matmul": "double_buffered"}
    if ring:
        options["ring"] = ring
    ring_graph = mc.Compiled(path=mc.graph_path("mlp_gelu"), dims=dims, options=options)
    two = mc.Compiled(path=mc.graph_path("mlp_gelu"), dims=dims, options={"matmul": "vectorized"})
    sources = "\n".join(ring_graph.kernel_sources)
    assert f"mc_gemm_f32_ring<{config}>" in sources, ring_graph.launch_names
    assert ring_graph.kernel_launches == 2
    inputs = uniform_inputs(oracle, ring_graph.input_sizes, 1)
    x, y = ring_graph.run(inputs), two.run(inputs)
    for p, q in zip(x, y):
        assert np.array_equal(p.view(np.uint32), q.view(np.uint32))


@pytest.mark.parametrize("config", ["wide", "wide8", "mid", "thin", "big"])
def test_a_fused_group_on_ragged_ring_tiles_gives_the_unfused_bits(device, mc, oracle, config):
    # M = 1000 leaves the last row of tiles ragged on every configuration:
    # the store skips the rows past M (with one or two columns per lane the
    # epilogue runs over a batch of rows first, and reads no operand for
    # those rows). Fused and unfused graphs give the same bits, within the
    # graph tolerance of the oracle.
    print(f"case ragged fused ring {config}", flush=True)
    dims = {"M": 1000, "K": 512, "N": 1024}
    opts = {"matmul": "double_buffered", "ring": config}
    fused = mc.Compiled(path=mc.graph_path("matmul_bias_relu"), dims=dims, options=opts)
    plain = mc.Compiled(path=mc.graph_path("matmul_bias_relu"), dims=dims, options={**opts, "epilogue": 0})
    assert any(len(ids) > 1 for ids in fused.launch_nodes), fused.launch_names
    inputs = uniform_inputs(oracle, fused.input_sizes, 5)
    x, y = fused.run(inputs), plain.run(inputs)
    for p, q in zip(x, y):
        assert np.array_equal(p.view(np.uint32), q.view(np.uint32)), config
    cpu = oracle.evaluate_compiled(fused, inputs)
    for p, c in zip(x, cpu):
        assert_close(p, c, 1e-4, 1e-4 * max(1.0, max_abs(c)), config)


# Every ring configuration forced (mc_launch_matmul_cfg, as the autotuner
# launches them), unsplit and split: the same bits as each other (each C
# element gets the same MFMA sequence whatever the tile), and within the
# dot-product bound, as is the plan's own choice (which may be the
# narrow-tile body for split_k, whose accumulation order is its own).
# Ragged M and N, thin and mid tiles at M > 32, a single mid tile with a
# long K, and split counts that do and do not divide K's steps evenly.
FORCED_SHAPES = [(300, 96, 260), (1000, 512, 1028), (64, 2048, 128), (33, 256, 4100)]


def run_cfg(mc, kernel, ring, da, db, m, n, k, splits, ws):
    dc = mc.DeviceBuffer.from_array(np.full(m * n + GUARD, np.nan, dtype=np.float32))
    mc.launch_matmul_cfg(kernel, da.ptr, db.ptr, dc.ptr, m, n, k, None, splits, ws.ptr if ws else None, ring)
    mc.synchronize()
    out = dc.download()
    assert np.all(np.isnan(out[m * n:])), f"{ring}: a write past the end of C"
    assert not np.any(np.isnan(out[:m * n])), f"{ring}: an element of C was not written"
    return out[:m * n]


@pytest.mark.parametrize("splits", [1, 3, 8])
@pytest.mark.parametrize("m,k,n", FORCED_SHAPES)
def test_forced_ring_configurations_give_the_plans_bits(device, mc, oracle, m, k, n, splits):
    print(f"case forced ring {m}x{k}x{n} splits {splits}", flush=True)
    a = oracle.uniform(m * k, 21, -1.0, 1.0)
    b = oracle.uniform(k * n, 22, -1.0, 1.0)
    da, db = mc.DeviceBuffer.from_array(a), mc.DeviceBuffer.from_array(b)
    kernel = "split_k" if splits > 1 else "double_buffered"
    ws_bytes = mc.matmul_workspace_bytes(kernel, m, n, splits) if splits > 1 else 0
    ws = mc.DeviceBuffer(ws_bytes) if ws_bytes else None
    ref = run_cfg(mc, kernel, "wide", da, db, m, n, k, splits, ws)
    for ring in ("mid", "big", "thin", "wide8"):
        got = run_cfg(mc, kernel, ring, da, db, m, n, k, splits, ws)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), ring
    exact, absdot = oracle.gemm_f64(a, b, m, k, n)
    bound = fp32_gemm_bound(exact, absdot, k)
    assert np.all(np.abs(ref.astype(np.float64) - exact) <= bound)
    planned = run_cfg(mc, kernel, "auto", da, db, m, n, k, splits, ws)
    assert np.all(np.abs(planned.astype(np.float64) - exact) <= bound)


def test_split_k_runs_unsplit_on_two_64x64_narrow_tiles_per_cu_where_they_fit(device, mc, oracle):
    # 1024x512x2048 (m, k, n): the split rule asks for 2 splits on 256 CUs;
    # 64x64 narrow tiles number 512, two per CU, so the split_k rung runs it
    # unsplit on them: the bits of a forced narrow launch (the same plan),
    # not those of the rule's two splits on the ring, within the dot-product
    # bound.
    m, k, n = 1024, 512, 2048
    if int(device["cu_count"]) != 256:
        pytest.skip("tile counts are for 256 CUs")
    splits = mc.matmul_splits("split_k", m, n, k, 256)
    assert splits == 2
    a = oracle.uniform(m * k, 23, -1.0, 1.0)
    b = oracle.uniform(k * n, 24, -1.0, 1.0)
    da, db = mc.DeviceBuffer.from_array(a), mc.DeviceBuffer.from_array(b)
    ws = mc.DeviceBuffer(mc.matmul_workspace_bytes("split_k", m, n, splits))
    planned = run_cfg(mc, "split_k", "auto", da, db, m, n, k, splits, ws)
    narrow = run_cfg(mc, "split_k", "narrow", da, db, m, n, k, splits, ws)
    assert np.array_equal(planned.view(np.uint32), narrow.view(np.uint32))
    split = run_cfg(mc, "split_k", "wide", da, db, m, n, k, splits, ws)
    assert not np.array_equal(planned.view(np.uint32), split.view(np.uint32))
    rows = np.arange(0, m, 7)
    exact, absdot = oracle.gemm_f64(a.reshape(m, k)[rows].ravel(), b, rows.size, k, n)
    assert np.all(np.abs(planned.reshape(m, n)[rows].astype(np.float64).ravel() - exact) <=
                  fp32_gemm_bound(exact, absdot, k))


def test_a_forced_configuration_the_product_cannot_take_is_an_error(device, mc):
    # K not a multiple of 32: no ring configuration runs it.
    da, db, dc = mc.DeviceBuffer(4 * 64 * 40), mc.DeviceBuffer(4 * 40 * 64), mc.DeviceBuffer(4 * 64 * 64)
    with pytest.raises(mc.HipError):
        mc.launch_matmul_cfg("double_buffered", da.ptr, db.ptr, dc.ptr, 64, 64, 40, None, 1, None, "mid")


def test_an_unfused_product_with_a_tile_per_cu_takes_the_8_wave_block_with_the_same_bits(device, mc, oracle):
    # 2048^3 double_buffered: 256 tiles of 128x128 on 256 CUs run as one
    # 8-wave block each (wide8); forced wide (4-wave blocks) and the
    # two-stage body give the same bits, and a fused graph of the same
    # product with ring=wide8 compiles the 8-wave body.
    m = n = k = 2048
    if int(device["cu_count"]) != 256:
        pytest.skip("tile counts are for 256 CUs")
    a = oracle.uniform(m * k, 25, -1.0, 1.0)
    b = oracle.uniform(k * n, 26, -1.0, 1.0)
    da, db = mc.DeviceBuffer.from_array(a), mc.DeviceBuffer.from_array(b)
    planned = run_cfg(mc, "double_buffered", "auto", da, db, m, n, k, 1, None)
    for ring in ("wide8", "wide"):
        got = run_cfg(mc, "double_buffered", ring, da, db, m, n, k, 1, None)
        assert np.array_equal(got.view(np.uint32), planned.view(np.uint32)), ring
    two = run(mc, "vectorized", da, db, m, n, k)
    assert np.array_equal(two.view(np.uint32), planned.view(np.uint32))
    g = mc.Compiled(path=mc.graph_path("matmul_bias_relu"), dims={"M": m, "K": k, "N": n},
                    options={"matmul": "double_buffered", "ring": "wide8"})
    assert "mc_gemm_f32_ring<McRingWide8>" in "\n".join(g.kernel_sources), g.launch_names


def test_the_ring_option_gives_one_set_of_bits_for_every_ring_configuration(device, mc, oracle):
    # ring=wide|mid|thin on the MLP at B=1024 (GEMM1 split in two, GEMM2 in
    # eight, each with its group fused into the store or the split sum): the
    # same bits for each, and the planner's choice (the narrow-tile body for
    # GEMM2) within the graph tolerance of the oracle.
    dims = {"B": 1024}
    ref = mc.Compiled(path=mc.graph_path("mlp_gelu"), dims=dims, options={"ring": "wide"})
    inputs = uniform_inputs(oracle, ref.input_sizes, 3)
    want = ref.run(inputs)
    planned = mc.Compiled(path=mc.graph_path("mlp_gelu"), dims=dims)
    cpu = oracle.evaluate_compiled(planned, inputs)[0]
    assert_close(planned.run(inputs)[0], cpu, 1e-4, 1e-4 * max(1.0, max_abs(cpu)), "planner's choice")
    for ring in ("mid", "thin"):
        print(f"case ring option {ring}", flush=True)
        c = mc.Compiled(path=mc.graph_path("mlp_gelu"), dims=dims, options={"ring": ring})
        assert c.matmul_kernels == ref.matmul_kernels
        got = c.run(inputs)
        for p, q in zip(got, want):
            assert np.array_equal(p.view(np.uint32), q.view(np.uint32)), ring
        c.close()
    with pytest.raises(mc.MinicompilerError):
        mc.Compiled(path=mc.graph_path("mlp_gelu"), dims=dims, options={"ring": "huge"})


@pytest.mark.parametrize("m,k,n,splits", [(256, 2048, 256, 8), (16, 4096, 1024, 4)])
def test_split_k_with_a_workspace_off_16_bytes_gives_the_aligned_bits(device, mc, oracle, m, k, n, splits):
    # The ring body writes partials 4-16 bytes at a time, so a workspace that
    # is not 16-byte aligned (a C-ABI caller may pass one) must send the
    # product to the two-stage body, whose scalar stores give the same bits;
    # the narrow-tile body (the plan's choice for 256x2048x256) stores such
    # partials float by float. Either way the bits do not depend on where
    # the workspace is.
    print(f"case split_k unaligned workspace {m}x{k}x{n} splits={splits}", flush=True)
    a = oracle.uniform(m * k, 21, -1.0, 1.0)
    b = oracle.uniform(k * n, 22, -1.0, 1.0)
    da, db = mc.DeviceBuffer.from_array(a), mc.DeviceBuffer.from_array(b)
    ws_bytes = mc.matmul_workspace_bytes("split_k", m, n, splits)
    ws = mc.DeviceBuffer(ws_bytes + 64)
    outs = []
    for offset in (0, 4, 8):
        dc = mc.DeviceBuffer.from_array(np.full(m * n, np.nan, dtype=np.float32))
        mc.launch_matmul("split_k", da.ptr, db.ptr, dc.ptr, m, n, k, None, splits, ws.ptr + offset)
        mc.synchronize()
        outs.append(dc.download())
    for o in outs[1:]:
        assert np.array_equal(outs[0].view(np.uint32), o.view(np.uint32))
    exact, absdot = oracle.gemm_f64(a, b, m, k, n)
    assert np.all(np.abs(outs[0].astype(np.float64) - exact) <= fp32_gemm_bound(exact, absdot, k))
