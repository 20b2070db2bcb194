"""Products whose B is 2 GiB or more: the ring and narrow bodies address
their operands through buffer loads with 31-bit byte offsets from a tile's
origin, so the planners route these to the two-stage body, which addresses
with 64-bit pointers. The result must still be within the reference's
dot-product bound (tests/test_cuda_backend.cpp:119-162) on sampled
elements, with no write past the end of C."""

import numpy as np
import pytest

from helpers import fp32_gemm_bound

pytestmark = pytest.mark.gpu

GUARD = 4096


@pytest.mark.parametrize("kernel,splits", [("double_buffered", 1), ("split_k", 4)])
def test_a_2_gib_operand_takes_a_64_bit_body_and_stays_in_bound(device, mc, oracle, kernel, splits):
    m, k, n = 16, 32768, 16384  # B: 32768 x 16384 fp32 = 2 GiB
    print(f"case large operands {kernel} {m}x{k}x{n} splits={splits}", flush=True)
    a = oracle.uniform(m * k, 51, -1.0, 1.0)
    b = oracle.uniform(k * n, 52, -1.0, 1.0)
    da, db = mc.DeviceBuffer.from_array(a), mc.DeviceBuffer.from_array(b)
    ws = mc.DeviceBuffer(mc.matmul_workspace_bytes(kernel, m, n, splits)) if splits > 1 else None
    dc = mc.DeviceBuffer.from_array(np.full(m * n + GUARD, np.nan, dtype=np.float32))
    mc.launch_matmul(kernel, da.ptr, db.ptr, dc.ptr, m, n, k, None, splits, ws.ptr if ws else None)
    mc.synchronize()
    out = dc.download()
    assert np.all(np.isnan(out[m * n:])), "a write past the end of C"
    got = out[:m * n]
    assert not np.any(np.isnan(got)), "an element of C was not written"
    rng = np.random.default_rng(7)
    rows, cols = rng.integers(0, m, 1000), rng.integers(0, n, 1000)
    exact, absdot = oracle.gemm_f64_sampled(a, b, rows, cols, k, n)
    g = got.astype(np.float64)[rows * n + cols]
    bad = np.abs(g - exact) > fp32_gemm_bound(exact, absdot, k)
    assert not np.any(bad), f"{np.count_nonzero(bad)} of 1000 sampled elements outside the bound"
