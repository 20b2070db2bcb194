"""The FP32 ring body against the two-stage body, through the C ABI.

double_buffered and split_k run the ring body (gemm_f32_ring.h) when K is a
multiple of 32 and N of 4; vectorized always runs the two-stage body
(gemm_f32_mfma.h, one stage). Both accumulate every C element by the same
v_mfma_f32_32x32x2_f32 sequence, so the outputs must be identical bit for
bit, and within the reference's dot-product bound
(tests/test_cuda_backend.cpp:119-162). The shapes reach both ring
configurations on a 256-CU MI355X: two blocks per CU when there are at least
two 128x128 tiles per CU, one 8-wave block per CU otherwise; blocks that take
two tiles; ragged edges; a grid that is not a multiple of 8."""

import numpy as np
import pytest

from helpers import fp32_gemm_bound, uniform_inputs

pytestmark = pytest.mark.gpu

GUARD = 4096  # floats after C, prefilled with NaN; must stay untouched

# (m, k, n): 544 tiles (two per CU, some blocks take two tiles), ragged M and N;
# 304 tiles (one 8-wave block per CU, some take two); 9 tiles (grid of 9);
# 256 tiles, one each (the class of the MLP's second GEMM); one row, one K step.
SHAPES = [(4000, 64, 2052), (2048, 96, 2432), (300, 96, 260), (8192, 256, 512), (1, 32, 4)]


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


def test_fused_epilogue_on_the_two_per_cu_ring_equals_the_two_stage_body(device, mc, oracle):
    # The MLP block at B=4096: GEMM1 (4096x2048x512, 512 tiles) runs the ring
    # with two blocks per CU and bias+GELU fused into its store; GEMM2
    # (4096x512x2048, 128 tiles) the one-block ring. The vectorized graph runs
    # the two-stage body (also fused): identical bits throughout.
    dims = {"B": 4096}
    ring = mc.Compiled(path=mc.graph_path("mlp_gelu"), dims=dims, options={"matmul": "double_buffered"})
    two = mc.Compiled(path=mc.graph_path("mlp_gelu"), dims=dims, options={"matmul": "vectorized"})
    sources = "\n".join(ring.kernel_sources)
    assert "mc_gemm_f32_ring<McRingWide>" in sources, ring.launch_names
    assert any(len(ids) > 1 for ids in ring.launch_nodes)
    inputs = uniform_inputs(oracle, ring.input_sizes, 1)
    x, y = ring.run(inputs), two.run(inputs)
    for p, q in zip(x, y):
        assert np.array_equal(p.view(np.uint32), q.view(np.uint32))
