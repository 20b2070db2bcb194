"""The bf16/fp16 matrix-core GEMM on inputs already stored as 16-bit values
(BASELINE config 5's mode) against float64 dot products, through the C ABI.
Shapes with K a multiple of 64 and N a multiple of 8 take the 256x256 tile
path with direct-to-LDS loads and transposed LDS reads; the others take the
general kernel. Bounds are the reference's tensor-core bound
(tests/test_cuda_backend.cpp:164-219) and, against the product of the
already-rounded inputs, the FP32 accumulation bound."""

import numpy as np
import pytest

from helpers import U32, gamma, lowp_gemm_bound

pytestmark = pytest.mark.gpu

FORMATS = [("tensor_core_bf16", 1, 2.0 ** -8, False), ("tensor_core_f16", 2, 2.0 ** -11, True)]
# (m, k, n): tile-aligned, ragged M, ragged N (multiple of 8), tiny, several K tiles, a non-multiple-of-8 N and a
# K that is not a multiple of 64 (general kernel). The fast kernel stores C as 8-row by 32-column pieces: the
# ragged shapes put the matrix edge at every offset within one (M % 16 = 12, 15, 8, 1; N % 32 = 8, 24, 16).
SHAPES = [(256, 64, 256), (300, 128, 264), (1, 64, 8), (513, 192, 1000), (512, 1024, 768), (96, 256, 4100),
          (200, 100, 136), (271, 128, 280), (264, 64, 272)]
GUARD = 4096  # floats after C, prefilled with NaN; must stay untouched


def run_lowp(mc, oracle, kernel, dtype, a32, b32, m, k, n):
    da, db = mc.DeviceBuffer.from_array(a32), mc.DeviceBuffer.from_array(b32)
    ha, hb = mc.DeviceBuffer(2 * m * k), mc.DeviceBuffer(2 * k * n)
    mc.convert_f32(dtype, da.ptr, ha.ptr, m * k)
    mc.convert_f32(dtype, db.ptr, hb.ptr, k * n)
    c = mc.DeviceBuffer.from_array(np.full(m * n + GUARD, np.nan, dtype=np.float32))
    mc.launch_matmul_lowp(kernel, dtype, ha.ptr, hb.ptr, c.ptr, m, n, k)
    mc.synchronize()
    out = c.download()
    assert np.all(np.isnan(out[m * n:])), "a write past the end of C"
    return out[:m * n].astype(np.float64)


@pytest.mark.parametrize("kernel,dtype,u,subnormals", FORMATS)
@pytest.mark.parametrize("m,k,n", SHAPES)
def test_pre_cast_gemm_is_within_the_precision_bounds(device, mc, oracle, kernel, dtype, u, subnormals, m, k, n):
    print(f"case {kernel} {m}x{k}x{n}", flush=True)
    a32 = oracle.uniform(m * k, 7, -1.0, 1.0)
    b32 = oracle.uniform(k * n, 8, -1.0, 1.0)
    gpu = run_lowp(mc, oracle, kernel, dtype, a32, b32, m, k, n)
    assert not np.any(np.isnan(gpu)), "an element of C was not written"
    exact, absdot = oracle.gemm_f64(a32, b32, m, k, n)
    assert np.all(np.abs(gpu - exact) <= lowp_gemm_bound(exact, absdot, k, u, subnormals))
    rnd = oracle.round_bf16 if dtype == 1 else oracle.round_f16
    ex2, ab2 = oracle.gemm_f64(rnd(a32), rnd(b32), m, k, n)
    assert np.all(np.abs(gpu - ex2) <= gamma(k) * ab2 + 2 * U32 * np.abs(ex2) + 1e-30)


@pytest.mark.parametrize("kernel,dtype,u,subnormals", FORMATS)
def test_pre_cast_gemm_at_8192_cubed_on_sampled_elements(device, mc, oracle, kernel, dtype, u, subnormals):
    # BASELINE config 5's square shape; 2000 sampled elements against float64
    # (bench/bench_cuda.cpp:386-413), plus the NaN prefill of every element.
    m = n = k = 8192
    print(f"case {kernel} 8192^3", flush=True)
    a32 = oracle.uniform(m * k, 1, -1.0, 1.0)
    b32 = oracle.uniform(k * n, 2, -1.0, 1.0)
    gpu = run_lowp(mc, oracle, kernel, dtype, a32, b32, m, k, n)
    assert not np.any(np.isnan(gpu))
    rng = np.random.default_rng(5)
    rows, cols = rng.integers(0, m, 2000), rng.integers(0, n, 2000)
    rnd = oracle.round_bf16 if dtype == 1 else oracle.round_f16
    ex2, ab2 = oracle.gemm_f64_sampled(rnd(a32), rnd(b32), rows, cols, k, n)
    got = gpu[rows * n + cols]
    assert np.all(np.abs(got - ex2) <= gamma(k) * ab2 + 2 * U32 * np.abs(ex2) + 1e-30)
    exact, absdot = oracle.gemm_f64_sampled(a32, b32, rows, cols, k, n)
    assert np.all(np.abs(got - exact) <= lowp_gemm_bound(exact, absdot, k, u, subnormals))
    # BASELINE's own tolerance against the unrounded fp32 inputs: sqrt(K) 2^-8 max|a| max|b|.
    assert np.max(np.abs(got - exact)) <= np.sqrt(k) * (2.0 ** -8 if dtype == 1 else 2.0 ** -11)


# On 256 CUs: 6 and 1 tiles of 256x256 (each run as two 128-row halves),
# then 272 tiles with M ragged (256 whole tiles and the last 16 as halves,
# the second half of each partly past M).
GRAPH_SHAPES = [(300, 256, 520), (256, 512, 256), (64, 64, 8), (4300, 64, 4096)]


@pytest.mark.parametrize("kernel", ["tensor_core_bf16", "tensor_core_f16"])
@pytest.mark.parametrize("m,k,n", GRAPH_SHAPES)
def test_graph_tensor_core_matmuls_convert_then_run_the_fast_kernel_bit_for_bit(device, mc, oracle, kernel, m, k, n):
    # A compiled graph rounds fp32 operands to 16 bits into workspace (a
    # constant weight once, the input per run) and runs the 256x256 kernel:
    # the same bits as the kernel that rounds while staging, with K unsplit;
    # with a bias+GELU group fused into its store, the same bits as the
    # separate kernels.
    print(f"case {kernel} {m}x{k}x{n}", flush=True)
    text = (f"input x : f32[{m}, {k}]\nconst w : f32[{k}, {n}] = uniform(seed=2, lo=-1, hi=1)\n"
            f"const bias : f32[{n}] = uniform(seed=3, lo=-0.01, hi=0.01)\nconst half : f32[] = 0.5\n"
            "const one : f32[] = 1.0\nconst c : f32[] = 0.7978846\nconst coef : f32[] = 0.044715\n"
            "h = matmul x, w\nhb = add h, bias\nx2 = mul hb, hb\nx3 = mul x2, hb\nt = mul x3, coef\n"
            "u0 = add hb, t\nu = mul u0, c\nth = tanh u\np = add th, one\nhh = mul hb, half\ny = mul hh, p\noutput y\n")
    x = oracle.uniform(m * k, 1, -1.0, 1.0)
    runs = {}
    for name, opts in (("fast+fused", {}), ("fast", {"epilogue": 0})):
        c = mc.Compiled(text, options={"matmul": kernel, **opts})
        assert c.matmul_kernels == [kernel]
        runs[name] = (c, c.run([x])[0])
    assert any(len(ids) > 1 for ids in runs["fast+fused"][0].launch_nodes)
    assert np.array_equal(runs["fast+fused"][1].view(np.uint32), runs["fast"][1].view(np.uint32))
    # The GEMM alone (weights an input, converted per run) against the
    # operator-level staging kernel on the same fp32 operands, one split:
    # the same rounding and the same accumulation order, so identical bits.
    mm = f"input x : f32[{m}, {k}]\ninput w : f32[{k}, {n}]\nh = matmul x, w\noutput h\n"
    w = oracle.uniform(k * n, 9, -1.0, 1.0)
    g32 = mc.Compiled(mm, options={"matmul": kernel}).run([x, w])[0]
    dx, dw = mc.DeviceBuffer.from_array(x), mc.DeviceBuffer.from_array(w)
    dc = mc.DeviceBuffer.from_array(np.full(m * n, np.nan, np.float32))
    mc.launch_matmul(kernel, dx.ptr, dw.ptr, dc.ptr, m, n, k)
    mc.synchronize()
    assert np.array_equal(g32.view(np.uint32), dc.download().view(np.uint32)), "staging kernel"
    # And within the precision bound of the bf16/fp16 product against float64.
    g = g32.astype(np.float64)
    u, sub = (2.0 ** -8, False) if "bf16" in kernel else (2.0 ** -11, True)
    exact, absdot = oracle.gemm_f64(x, w, m, k, n)
    assert np.all(np.abs(g - exact) <= lowp_gemm_bound(exact, absdot, k, u, sub))
