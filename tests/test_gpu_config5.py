"""BASELINE config 5 at its full sizes: the bf16/fp16 matrix-core GEMM with
fp32 accumulation on the FFN shape 4096x14336x4096, and the GEMM with the
bias + GELU epilogue fused into its store (matmul_bias_gelu.mcg) at 8192^3
and at the FFN shape, with both 16-bit formats, on the inputs bench.py times.

Bounds (u = 2^-8 for bf16, 2^-11 for fp16; L = 1.13 bounds the slope of
gelu_tanh, whose derivative peaks at 1.1289 near x = 1.5):
- the reference's tensor-core bound against float64 on the unrounded inputs,
  (2u + u^2 + 2 gamma_K) sum|ab| + 2 u32 |exact| (+ fp16 subnormal loss),
  tests/test_cuda_backend.cpp:164-219;
- BASELINE's own tolerance against the fp32 reference on the unrounded
  inputs: sqrt(K) u max|a| max|b| (times L after the GELU);
- against float64 on the already-rounded inputs: the FP32 accumulation bound
  gamma_K sum|ab| + u32 |exact| (times L after the GELU, plus the fused
  group's rtol 1e-5), which isolates accumulation and epilogue from input
  rounding.
Rows of a product are independent, so the epilogue graph is checked on its
first and last 256 rows (the first and the last tile row) and on two seeded
256-row blocks in between (each straddling a tile boundary) against the
oracle run on those rows alone; the bare GEMM on 2000 sampled elements
(bench/bench_cuda.cpp:386-413). Every output is prefilled with NaN on the
device (the graph's output is bound to a 0xFF-filled buffer) and checked
for unwritten elements everywhere."""

import os

import numpy as np
import pytest

from helpers import U32, gamma, lowp_gemm_bound, row_blocks, run_into_prefilled

pytestmark = pytest.mark.gpu

FORMATS = [("tensor_core_bf16", 1, 2.0 ** -8, False), ("tensor_core_f16", 2, 2.0 ** -11, True)]
GELU_SLOPE = 1.13
GUARD = 4096


@pytest.fixture
def threaded_oracle(oracle):
    """The oracle on the host's share of cores (at most 16) for these sizes."""
    oracle.set_threads(max(1, min(os.cpu_count() or 1, 16)))
    yield oracle
    oracle.set_threads(1)


def gelu_tanh_f64(h: np.ndarray) -> np.ndarray:
    c = np.sqrt(2.0 / np.pi)
    return 0.5 * h * (1.0 + np.tanh(c * (h + 0.044715 * h * h * h)))


@pytest.mark.parametrize("kernel,dtype,u,subnormals", FORMATS)
def test_pre_cast_gemm_on_the_ffn_shape_on_sampled_elements(device, mc, threaded_oracle, kernel, dtype, u,
                                                             subnormals):
    oracle = threaded_oracle
    m, k, n = 4096, 4096, 14336
    print(f"case {kernel} ffn {m}x{k}x{n}", flush=True)
    a32 = oracle.uniform(m * k, 1, -1.0, 1.0)
    b32 = oracle.uniform(k * n, 2, -1.0, 1.0)
    da, db = mc.DeviceBuffer.from_array(a32), mc.DeviceBuffer.from_array(b32)
    ha, hb = mc.DeviceBuffer(2 * m * k), mc.DeviceBuffer(2 * k * n)
    mc.convert_f32(dtype, da.ptr, ha.ptr, m * k)
    mc.convert_f32(dtype, db.ptr, hb.ptr, k * n)
    del da, db
    c = mc.DeviceBuffer.from_array(np.full(m * n + GUARD, np.nan, dtype=np.float32))
    mc.launch_matmul_lowp(kernel, dtype, ha.ptr, hb.ptr, c.ptr, m, n, k)
    mc.synchronize()
    out = c.download()
    assert np.all(np.isnan(out[m * n:])), "a write past the end of C"
    gpu = out[:m * n].astype(np.float64)
    assert not np.any(np.isnan(gpu)), "an element of C was not written"
    rng = np.random.default_rng(11)
    # Sampled rows and columns, plus the corners of the last round of tiles
    # (the FFN shape's 896 tiles leave a partial round on 256 CUs).
    rows = np.concatenate([rng.integers(0, m, 2000), [0, m - 1, m - 1, 0]])
    cols = np.concatenate([rng.integers(0, n, 2000), [0, n - 1, 0, n - 1]])
    got = gpu[rows * n + cols]
    rnd = oracle.round_bf16 if dtype == 1 else oracle.round_f16
    ex2, ab2 = oracle.gemm_f64_sampled(rnd(a32), rnd(b32), rows, cols, k, n)
    assert np.all(np.abs(got - ex2) <= gamma(k) * ab2 + 2 * U32 * np.abs(ex2) + 1e-30)
    exact, absdot = oracle.gemm_f64_sampled(a32, b32, rows, cols, k, n)
    assert np.all(np.abs(got - exact) <= lowp_gemm_bound(exact, absdot, k, u, subnormals))
    assert np.max(np.abs(got - exact)) <= np.sqrt(k) * u


EPILOGUE_SHAPES = [(8192, 8192, 8192), (4096, 4096, 14336)]


@pytest.mark.parametrize("kernel,dtype,u,subnormals", FORMATS)
@pytest.mark.parametrize("m,k,n", EPILOGUE_SHAPES)
def test_gemm_with_fused_bias_gelu_matches_the_oracle_on_row_blocks(device, mc, threaded_oracle, kernel,
                                                                              dtype, u, subnormals, m, k, n):
    oracle = threaded_oracle
    rows = 256
    print(f"case {kernel} matmul_bias_gelu {m}x{k}x{n}", flush=True)
    dims = {"M": m, "K": k, "N": n}
    c = mc.Compiled(path=mc.graph_path("matmul_bias_gelu"), dims=dims, options={"matmul": kernel})
    assert c.matmul_kernels == [kernel]
    assert c.kernel_launches <= 2, "the bias + GELU group is fused into the GEMM's store"
    assert any(len(ids) > 1 for ids in c.launch_nodes)
    x = oracle.uniform(m * k, 1, -1.0, 1.0)
    gpu = run_into_prefilled(mc, c, [x])[0]
    assert not np.any(np.isnan(gpu)), f"{np.count_nonzero(np.isnan(gpu))} elements of y were not written"
    gpu = gpu.reshape(m, n)
    del c
    # The same graph on `rows` rows, passes only: its constants are seeded per
    # tensor, so w and bias equal the full graph's.
    part = mc.Compiled(path=mc.graph_path("matmul_bias_gelu"), dims={"M": rows, "K": k, "N": n}, backend="none")
    g = part.graph()
    consts = {nd["id"]: part.constant(nd["id"]) for nd in g["nodes"] if nd["op"] == oracle.CONSTANT}
    (mm,) = [nd for nd in g["nodes"] if nd["op"] == oracle.MATMUL]
    w = consts[mm["inputs"][1]]
    (bias,) = [v for v in consts.values() if v.size == n]
    rnd = oracle.round_bf16 if dtype == 1 else oracle.round_f16
    wr = rnd(w)
    xs = x.reshape(m, k)
    for first in row_blocks(m, rows, seed=m + n):
        print(f"  rows {first}..{first + rows - 1}", flush=True)
        got = gpu[first:first + rows].reshape(-1).astype(np.float64)
        xa = np.ascontiguousarray(xs[first:first + rows]).reshape(-1)
        # BASELINE's tolerance against the fp32 oracle on the unrounded inputs.
        cpu = oracle.evaluate(g, consts, [xa])[0].astype(np.float64)
        worst = float(np.max(np.abs(got - cpu)))
        assert worst <= GELU_SLOPE * np.sqrt(k) * u, f"rows {first}..: {worst} against the fp32 oracle"
        # The tensor-core bound against float64 on the unrounded inputs.
        exact, absdot = oracle.gemm_f64(xa, w, rows, k, n)
        hb = (exact.reshape(rows, n) + bias.astype(np.float64)).reshape(-1)
        y64 = gelu_tanh_f64(hb)
        scale = max(1.0, float(np.max(np.abs(y64))))
        fused_tol = 1e-5 * np.abs(y64) + 1e-5 * scale
        bound = GELU_SLOPE * (lowp_gemm_bound(exact, absdot, k, u, subnormals) + U32 * np.abs(hb)) + fused_tol
        bad = np.abs(got - y64) > bound
        assert not np.any(bad), f"rows {first}..: {np.count_nonzero(bad)} elements outside the tensor-core bound"
        # Accumulation and epilogue alone: float64 on the rounded inputs.
        ex2, ab2 = oracle.gemm_f64(rnd(xa), wr, rows, k, n)
        hb2 = (ex2.reshape(rows, n) + bias.astype(np.float64)).reshape(-1)
        y2 = gelu_tanh_f64(hb2)
        bound2 = GELU_SLOPE * (gamma(k) * ab2 + 2 * U32 * np.abs(hb2)) + 1e-5 * np.abs(y2) + 1e-5 * scale
        bad = np.abs(got - y2) > bound2
        assert not np.any(bad), f"rows {first}..: {np.count_nonzero(bad)} elements outside the accumulation bound"
