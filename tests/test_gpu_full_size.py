"""Parity at BASELINE's full sizes, on the inputs bench.py times.

- GELU [4096, 4096] and BatchNorm + ReLU [200704, 256]: every element against
  the CPU oracle at the fused tolerance, rtol 1e-5 plus 1e-5 of the output's
  scale (tests/test_cuda_backend.cpp:412-414).
- The MLP block at B=8192 (GEMM1 with bias + GELU fused into its store, GEMM2
  with b2 + residual): the rows of a batch are independent, so the oracle's
  output for B=256 rows of x is the B=8192 output of those rows. The output
  is bound to a device buffer prefilled with NaN and checked for unwritten
  elements everywhere; the first and the last 256 rows (the last tile row of
  both GEMMs) and two seeded blocks in between, each straddling a tile
  boundary, are checked at the FP32 graph tolerance, rtol 1e-4 plus 1e-4 of
  the scale.
- The FP32 GEMM sweep (config 4) with the kernel and split count that auto
  resolves to on this device, as launch_matmul runs them: 2000 sampled
  elements per shape (all elements for the two small outputs) against
  float64 dot products, within the dot-product bound (2 gamma_K sum|ab| plus
  the final roundings, tests/test_cuda_backend.cpp:119-162), after a NaN
  prefill of every element (bench/bench_cuda.cpp:386-413)."""

import numpy as np
import pytest

from helpers import assert_close, fp32_gemm_bound, max_abs, row_blocks, run_into_prefilled

pytestmark = pytest.mark.gpu


def test_gelu_4096_squared_matches_the_oracle_everywhere(device, mc, oracle):
    print("case full gelu_chain 4096x4096", flush=True)
    c = mc.Compiled(path=mc.graph_path("gelu_chain"), dims={"M": 4096, "N": 4096})
    assert c.kernel_launches == 1
    x = oracle.uniform(4096 * 4096, 1, -3.0, 3.0)
    gpu = run_into_prefilled(mc, c, [x])[0]
    cpu = oracle.evaluate_compiled(c, [x])[0]
    assert_close(gpu, cpu, 1e-5, 1e-5 * max(1.0, max_abs(cpu)), "gelu 4096^2")


def test_batchnorm_relu_at_200704_rows_matches_the_oracle_everywhere(device, mc, oracle):
    print("case full batchnorm_relu 200704x256", flush=True)
    c = mc.Compiled(path=mc.graph_path("batchnorm_relu"), dims={"R": 200704, "C": 256})
    assert c.kernel_launches == 1
    x = oracle.normal(200704 * 256, 1, 0.0, 1.0)
    gpu = run_into_prefilled(mc, c, [x])[0]
    cpu = oracle.evaluate_compiled(c, [x])[0]
    assert_close(gpu, cpu, 1e-5, 1e-5 * max(1.0, max_abs(cpu)), "batchnorm 200704x256")
    assert np.all(gpu >= 0.0), "relu output below zero"


def test_mlp_at_batch_8192_matches_the_oracle_on_row_blocks_after_a_nan_prefill(device, mc, oracle):
    print("case full mlp_gelu B=8192", flush=True)
    batch, d, rows = 8192, 512, 256
    c = mc.Compiled(path=mc.graph_path("mlp_gelu"), dims={"B": batch})
    assert c.kernel_launches == 2, "both GEMMs carry their groups"
    x = oracle.uniform(batch * d, 1, -1.0, 1.0)
    gpu = run_into_prefilled(mc, c, [x])[0]
    assert not np.any(np.isnan(gpu)), f"{np.count_nonzero(np.isnan(gpu))} elements of y were not written"
    gpu = gpu.reshape(batch, d)
    # The same graph at B=256: its constants are seeded per tensor, so they
    # equal the B=8192 graph's.
    part = mc.Compiled(path=mc.graph_path("mlp_gelu"), dims={"B": rows}, backend="none")
    xs = x.reshape(batch, d)
    for first in row_blocks(batch, rows, seed=batch):
        cpu = oracle.evaluate_compiled(part, [np.ascontiguousarray(xs[first:first + rows]).reshape(-1)])[0]
        got = gpu[first:first + rows].reshape(-1)
        assert_close(got, cpu, 1e-4, 1e-4 * max(1.0, max_abs(cpu)), f"mlp rows {first}..{first + rows - 1}")


# (m, k, n), and whether every element is checked.
GEMM_SHAPES = [(1024, 1024, 1024, False), (2048, 2048, 2048, False), (4096, 4096, 4096, False),
               (8192, 8192, 8192, False), (256, 16384, 256, True), (16, 4096, 4096, True)]


@pytest.mark.parametrize("m,k,n,full", GEMM_SHAPES)
def test_fp32_gemm_sweep_with_the_resolved_kernel_is_within_the_dot_product_bound(device, mc, oracle, m, k, n, full):
    cus = int(device["cu_count"])
    kernel = mc.resolve_matmul_kernel("auto", m, n, k, cus)
    splits = mc.matmul_splits(kernel, m, n, k, cus)
    print(f"case full fp32 gemm {m}x{k}x{n} {kernel} splits={splits}", flush=True)
    a32 = oracle.uniform(m * k, 1, -1.0, 1.0)
    b32 = oracle.uniform(k * n, 2, -1.0, 1.0)
    da, db = mc.DeviceBuffer.from_array(a32), mc.DeviceBuffer.from_array(b32)
    dc = mc.DeviceBuffer.from_array(np.full(m * n, np.nan, dtype=np.float32))
    ws_bytes = mc.matmul_workspace_bytes(kernel, m, n, splits)
    ws = mc.DeviceBuffer(ws_bytes) if ws_bytes > 0 else None
    mc.launch_matmul(kernel, da.ptr, db.ptr, dc.ptr, m, n, k, None, splits, ws.ptr if ws else None)
    mc.synchronize()
    gpu = dc.download().astype(np.float64)
    assert not np.any(np.isnan(gpu)), "an element of C was not written"
    if full:
        exact, absdot = oracle.gemm_f64(a32, b32, m, k, n)
        got = gpu
    else:
        rng = np.random.default_rng(m + 3 * k)
        rows, cols = rng.integers(0, m, 2000), rng.integers(0, n, 2000)
        exact, absdot = oracle.gemm_f64_sampled(a32, b32, rows, cols, k, n)
        got = gpu[rows * n + cols]
    bad = np.abs(got - exact) > fp32_gemm_bound(exact, absdot, k)
    assert not np.any(bad), f"{np.count_nonzero(bad)} elements outside the bound"
