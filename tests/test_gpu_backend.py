"""The HIP backend on the GPU against the CPU oracle, through the C ABI.
Restates the reference's tests/test_cuda_backend.cpp cases for gfx950."""

import concurrent.futures as futures

import numpy as np
import pytest

from graphgen import make_random_graph
from helpers import U32, all_close, assert_close, fp32_gemm_bound, gamma, lowp_gemm_bound, max_abs, uniform_inputs

pytestmark = pytest.mark.gpu

# Tolerances (tests/test_cuda_backend.cpp:62-72): + - * / neg relu are IEEE
# on both sides and must match bit for bit; the transcendental functions
# (ocml on the GPU, the C library in the oracle) within rtol 1e-6 plus one
# ulp at 1.0.
TRANS_RTOL = 1e-6
TRANS_ATOL = 1.2e-7
UNARY = ["neg", "exp", "log", "sqrt", "relu", "sigmoid", "tanh"]
BINARY = ["add", "sub", "mul", "div"]
PATTERNS = [((17, 33), (17, 33)), ((17, 32), ()), ((), (17, 33)), ((17, 32), (32,)), ((17, 33), (17, 1)),
            ((17, 1), (1, 33)), ((2, 3, 4), (3, 1)), ((5, 1, 6), (1, 4, 1))]


def shape_text(s):
    return "f32[" + ", ".join(str(d) for d in s) + "]"


def unary_graph(op, shape):
    return f"input x : {shape_text(shape)}\ny = {op} x\noutput y\n"


def binary_graph(op, sa, sb):
    return f"input a : {shape_text(sa)}\ninput b : {shape_text(sb)}\ny = {op} a, b\noutput y\n"


def matmul_graph(m, k, n):
    return f"input a : f32[{m}, {k}]\ninput w : f32[{k}, {n}]\ny = matmul a, w\noutput y\n"


def run_both(mc, oracle, text, inputs, passes="default", options=None):
    c = mc.Compiled(text, passes=passes, options=options)
    return c.run(inputs), oracle.evaluate_compiled(c, inputs), c


def test_device_is_a_gfx950(device, mc):
    print(device)
    assert device["arch"].startswith("gfx950"), device["arch"]
    assert device["cu_count"] > 0 and device["wave_size"] == 64
    assert device["peak_bandwidth_gbs"] > 0 and device["peak_fp32_gflops"] > 0
    # HBM3E on gfx950 (MI350X / MI355X): 8 TB/s published; the runtime's
    # memory clock and bus width give 8.19 TB/s at four transfers per clock.
    assert 7000 < device["peak_bandwidth_gbs"] < 9000, device["peak_bandwidth_gbs"]
    assert "hip" in mc.Compiled(unary_graph("neg", (4,)), backend="hip").backend


@pytest.mark.parametrize("shape", [(37, 29), (64, 64)])  # scalar path, then 16-byte path
@pytest.mark.parametrize("op", UNARY)
def test_unary_ops_match_the_cpu_oracle(device, mc, oracle, op, shape):
    lo = 0.01 if op in ("log", "sqrt") else -6.0
    inputs = uniform_inputs(oracle, [shape[0] * shape[1]], 11, lo, 6.0)
    gpu, cpu, c = run_both(mc, oracle, unary_graph(op, shape), inputs)
    exact = op in ("neg", "relu")
    assert_close(gpu[0], cpu[0], 0.0 if exact else TRANS_RTOL, 0.0 if exact else TRANS_ATOL, f"{op} {shape}")
    ref = oracle.evaluate_compiled(c, inputs, mode="reference")
    assert_close(gpu[0], ref[0], 0.0 if exact else TRANS_RTOL, 0.0 if exact else TRANS_ATOL, f"{op} vs double")


def test_tanh_over_a_dense_range_and_its_special_values(device, mc, oracle):
    # The generated kernels' own tanh (a polynomial below |x| = 0.625, exp2
    # and a reciprocal above) against the double evaluator, at the unary
    # tolerance; the threshold, tiny and huge values, +-0, +-inf and NaN.
    xs = np.concatenate([np.linspace(-12, 12, 48001, dtype=np.float32),
                         np.float32(0.625) * np.array([1 - 2**-23, 1, 1 + 2**-23], np.float32),
                         -np.float32(0.625) * np.array([1 - 2**-23, 1, 1 + 2**-23], np.float32),
                         np.array([0.0, -0.0, 1e-30, -1e-30, 1e-45, 2**-20, 45.0, -45.0, 1e30, -1e30], np.float32),
                         np.array([np.inf, -np.inf], np.float32)]).astype(np.float32)
    c = mc.Compiled(unary_graph("tanh", (xs.size,)))
    gpu = c.run([xs])[0]
    ref = oracle.evaluate_compiled(c, [xs], mode="reference")[0]
    assert_close(gpu, ref, TRANS_RTOL, TRANS_ATOL, "tanh")
    assert np.array_equal(np.signbit(gpu[xs == 0]), np.signbit(xs[xs == 0]))  # -0 stays -0
    c4 = mc.Compiled(unary_graph("tanh", (4,)))
    assert np.all(np.isnan(c4.run([np.full(4, np.nan, np.float32)])[0]))


def test_one_plus_tanh_in_a_fused_group_over_a_dense_range(device, mc):
    # A group's 1 + tanh(x) is emitted as 2 / (1 + 2^(-2 x log2 e)) (one
    # exp2, one reciprocal): against float64, within 4 ulp plus the exp2
    # argument's rounding (of the constant 2 log2(e) and of its product with
    # x: 2 |x| 2 log2(e) 2^-24, times ln 2, relative), with no cancellation
    # as tanh(x) -> -1; +-inf and NaN as 1 + tanh gives them.
    xs = np.concatenate([np.linspace(-60, 60, 96001, dtype=np.float32),
                         np.array([0.0, -0.0, 1e-30, -1e-30, 1e30, -1e30, np.inf, -np.inf], np.float32)])
    c = mc.Compiled(f"input x : f32[{xs.size}]\nconst one : f32[] = 1.0\nt = tanh x\ny = add t, one\noutput y\n")
    (src,) = c.kernel_sources
    assert "mc_one_plus_tanh(r" in src and "mc_tanh(" not in src
    gpu = c.run([xs])[0].astype(np.float64)
    x64 = xs.astype(np.float64)
    with np.errstate(over="ignore"):
        ref = 2.0 / (1.0 + np.exp(-2.0 * x64))  # = 1 + tanh(x), without float64's own cancellation
    fin = np.isfinite(x64)
    bound = (4 * 2.0**-24 + 2 * np.abs(np.where(fin, x64, 0.0)) * 2.0 * np.log2(np.e) * 2.0**-24 * np.log(2)) * ref + 1e-37
    bad = np.where(fin, np.abs(gpu - ref) > bound, gpu != ref)  # 1 + tanh(+-inf) = 2, 0 exactly
    assert not np.any(bad), (xs[bad][:5], gpu[bad][:5], ref[bad][:5])
    nan = mc.Compiled("input x : f32[4]\nconst one : f32[] = 1.0\nt = tanh x\ny = add t, one\noutput y\n")
    assert np.all(np.isnan(nan.run([np.full(4, np.nan, np.float32)])[0]))


def test_halved_one_plus_tanh_equals_the_unhalved_form_bit_for_bit(device, mc):
    # GELU's tail (x * 0.5)(1 + tanh u) is emitted as x * mc_half_one_plus_tanh(u)
    # = x / (1 + 2^(-2 u log2 e)): the same bits as (x / 2) times the
    # mc_one_plus_tanh form wherever x / 2 is exact. The second graph also
    # outputs x * 0.5, which puts it in a kernel of its own, so its group
    # multiplies the loaded half by mc_one_plus_tanh.
    xs = np.concatenate([np.linspace(-60, 60, 96001, dtype=np.float32),
                         np.array([0.0, -0.0, 1e-30, -1e-30, 1e30, -1e30, np.inf, -np.inf, np.nan], np.float32)])
    head = f"input x : f32[{xs.size}]\nconst one : f32[] = 1.0\nconst half : f32[] = 0.5\n"
    body = "t = tanh x\np = add t, one\nh = mul x, half\ny = mul h, p\noutput y\n"
    fused = mc.Compiled(head + body)
    assert any("mc_half_one_plus_tanh(" in s for s in fused.kernel_sources)
    split = mc.Compiled(head + body + "output h\n")
    assert not any("mc_half_one_plus_tanh(" in s for s in split.kernel_sources)
    assert any("mc_one_plus_tanh(" in s for s in split.kernel_sources)
    a = fused.run([xs])[0]
    b = split.run([xs])[0]
    nan = np.isnan(a)
    assert np.array_equal(nan, np.isnan(b))
    assert np.array_equal(a[~nan].view(np.uint32), b[~nan].view(np.uint32))
    # And against float64: x / (1 + e^(-2x)), within the bound of the form
    # above, plus 6e-37 absolute: the reciprocal returns 0 where it would be
    # below the smallest normal float (for x below about -43.67), so the form
    # returns -0 where the exact value is below 5.2e-37 in magnitude.
    x64 = xs.astype(np.float64)
    fin = np.isfinite(x64)
    with np.errstate(over="ignore", invalid="ignore"):
        ref = x64 / (1.0 + np.exp(-2.0 * x64))
    bound = (5 * 2.0**-24 + 2 * np.abs(np.where(fin, x64, 0.0)) * 2.0 * np.log2(np.e) * 2.0**-24 * np.log(2)) \
        * np.abs(np.where(fin, ref, 0.0)) + 6e-37
    bad = fin & (np.abs(a.astype(np.float64) - np.where(fin, ref, 0.0)) > bound)
    assert not np.any(bad), (xs[bad][:5], a[bad][:5], ref[bad][:5])


@pytest.mark.parametrize("sa,sb", PATTERNS)
def test_binary_ops_match_bit_for_bit_for_every_broadcast_pattern(device, mc, oracle, sa, sb):
    for op in BINARY:
        sizes = [int(np.prod(sa, dtype=np.int64)), int(np.prod(sb, dtype=np.int64))]
        inputs = uniform_inputs(oracle, sizes, 5, 0.5, 2.0)
        gpu, cpu, _ = run_both(mc, oracle, binary_graph(op, sa, sb), inputs)
        assert np.array_equal(gpu[0].view(np.uint32), cpu[0].view(np.uint32)), (op, sa, sb)


MATMUL_SHAPES = [(1, 1, 1), (3, 5, 7), (1, 1000, 1), (33, 257, 65), (65, 9, 63), (127, 129, 131), (128, 128, 128),
                 (129, 13, 129), (256, 256, 256), (16, 4099, 16), (513, 77, 259), (129, 132, 260), (300, 1004, 36),
                 (2, 12, 4)]
FP32_KERNELS = ["auto", "naive", "tiled", "register_tiled_128", "register_tiled_64", "vectorized",
                "double_buffered", "split_k"]


@pytest.mark.parametrize("kernel", FP32_KERNELS)
def test_every_matmul_kernel_is_within_the_dot_product_bound(device, mc, oracle, kernel):
    # tests/test_cuda_backend.cpp:119-162: both sides within gamma_k sum|ab|.
    for m, k, n in MATMUL_SHAPES:
        inputs = uniform_inputs(oracle, [m * k, k * n], 3)
        c = mc.Compiled(matmul_graph(m, k, n), options={"matmul": kernel})
        gpu = c.run(inputs)[0]
        cpu = oracle.matmul(inputs[0], inputs[1], m, k, n)
        exact, absdot = oracle.gemm_f64(inputs[0], inputs[1], m, k, n)
        bound = fp32_gemm_bound(cpu.astype(np.float64), absdot, k)
        err = np.abs(gpu.astype(np.float64) - cpu)
        assert np.all(err <= bound), f"{kernel} {m}x{k}x{n}: worst {np.max(err / np.maximum(bound, 1e-300))}"


LOWP = [("tensor_core_bf16", 2.0 ** -8, False), ("tensor_core_f16", 2.0 ** -11, True)]
TC_SHAPES = [(1, 1, 1), (3, 5, 7), (33, 257, 65), (127, 129, 131), (128, 128, 128), (129, 33, 129), (16, 4099, 16),
             (300, 1004, 36), (2, 12, 4), (256, 256, 256)]


@pytest.mark.parametrize("kernel,u,subnormals", LOWP)
def test_matrix_core_matmuls_are_within_their_precision_bounds(device, mc, oracle, kernel, u, subnormals):
    # tests/test_cuda_backend.cpp:164-219.
    for m, k, n in TC_SHAPES:
        inputs = uniform_inputs(oracle, [m * k, k * n], 3)
        c = mc.Compiled(matmul_graph(m, k, n), options={"matmul": kernel})
        assert c.matmul_kernels == [kernel]
        gpu = c.run(inputs)[0].astype(np.float64)
        exact, absdot = oracle.gemm_f64(inputs[0], inputs[1], m, k, n)
        bound = lowp_gemm_bound(exact, absdot, k, u, subnormals)
        assert np.all(np.abs(gpu - exact) <= bound), f"{kernel} {m}x{k}x{n}"
        # Against the fp32 product of the rounded inputs: only accumulation order differs.
        rnd = oracle.round_bf16 if "bf16" in kernel else oracle.round_f16
        ra, rb = rnd(inputs[0]), rnd(inputs[1])
        ex2, ab2 = oracle.gemm_f64(ra, rb, m, k, n)
        assert np.all(np.abs(gpu - ex2) <= gamma(k) * ab2 + 2 * U32 * np.abs(ex2) + 1e-30), f"{kernel} rounded-input bound"


def test_tf32_cannot_run_on_gfx950_and_fails_to_compile(device, mc):
    with pytest.raises(mc.MinicompilerError) as e:
        mc.Compiled(matmul_graph(64, 64, 64), options={"matmul": "tensor_core_tf32"})
    assert "tensor_core_tf32" in str(e.value) and "gfx950" in str(e.value)
    for kernel in ("tensor_core_bf16", "tensor_core_f16"):
        mc.Compiled(matmul_graph(64, 64, 64), options={"matmul": kernel})


@pytest.mark.parametrize("m,k,n", [(33, 1000, 65), (128, 2048, 512), (16, 4099, 16), (2, 12, 4), (129, 260, 132),
                                   (64, 5, 8)])
def test_split_k_is_within_the_bound_for_any_split_count(device, mc, oracle, m, k, n):
    # tests/test_cuda_backend.cpp:241-313, through the GEMM operator ABI with
    # NaN-prefilled outputs so an unwritten element fails.
    a = oracle.uniform(m * k, 7, -1.0, 1.0)
    b = oracle.uniform(k * n, 8, -1.0, 1.0)
    exact, absdot = oracle.gemm_f64(a, b, m, k, n)
    da, db = mc.DeviceBuffer.from_array(a), mc.DeviceBuffer.from_array(b)
    dc = mc.DeviceBuffer(m * n * 4)
    g = gamma(k)
    for kernel, u, sub in [("split_k", 0.0, False)] + LOWP:
        for splits in (1, 2, 3, 7, 16, 64):
            ws_bytes = mc.matmul_workspace_bytes(kernel, m, n, splits)
            ws = mc.DeviceBuffer(ws_bytes) if ws_bytes else None
            dc.fill_bytes(0xFF)
            mc.launch_matmul(kernel, da.ptr, db.ptr, dc.ptr, m, n, k, None, splits, ws.ptr if ws else None)
            mc.synchronize()
            c = dc.download().astype(np.float64)
            if u == 0.0:
                bound = g * absdot + U32 * np.abs(exact)
            else:
                bound = lowp_gemm_bound(exact, absdot, k, u, sub)
            assert np.all(np.abs(c - exact) <= bound), f"{kernel} {m}x{k}x{n} splits={splits}"


def test_unresolved_auto_and_missing_workspace_are_errors(device, mc):
    d = mc.DeviceBuffer(64 * 64 * 4)
    with pytest.raises(mc.HipError):
        mc.launch_matmul("auto", d.ptr, d.ptr, d.ptr, 64, 64, 64)
    with pytest.raises(mc.HipError):
        mc.launch_matmul("split_k", d.ptr, d.ptr, d.ptr, 64, 64, 4096, None, 8, None)
    with pytest.raises(mc.HipError):
        mc.launch_matmul("tensor_core_tf32", d.ptr, d.ptr, d.ptr, 64, 64, 64)


def test_compiled_graphs_report_the_matmul_kernel_for_each_shape(device, mc):
    cus = device["cu_count"]
    text = ("input x : f32[128, 512]\ninput w1 : f32[512, 2048]\ninput w2 : f32[2048, 4096]\n"
            "h = matmul x, w1\ny = matmul h, w2\noutput y\n")
    c = mc.Compiled(text)
    assert c.matmul_kernels == [mc.resolve_matmul_kernel("auto", 128, 2048, 512, cus),
                                mc.resolve_matmul_kernel("auto", 128, 4096, 2048, cus)]
    c = mc.Compiled(matmul_graph(8, 8, 8), options={"matmul": "tiled"})
    assert c.matmul_kernels == ["tiled"]


@pytest.mark.parametrize("name,dims", [("gelu_chain", {"M": 64, "N": 300}),
                                       ("matmul_bias_relu", {"M": 33, "K": 70, "N": 129}),
                                       ("mlp_block_bn", {"B": 16, "D": 64, "H": 256}),
                                       ("mlp_gelu", {"B": 16, "D": 64, "H": 256}),
                                       ("batchnorm_relu", {"R": 49}),
                                       ("matmul_bias_gelu", {"M": 33, "K": 64, "N": 72})])
@pytest.mark.parametrize("passes", ["none", "default"])
def test_benchmark_graphs_match_the_cpu_oracle_fused_and_unfused(device, mc, oracle, name, dims, passes):
    # tests/test_cuda_backend.cpp:375-397: rtol 1e-5 plus 1e-5 of the output's scale.
    c = mc.Compiled(path=mc.graph_path(name), dims=dims, passes=passes)
    inputs = uniform_inputs(oracle, c.input_sizes, 1)
    gpu = c.run(inputs)
    cpu = oracle.evaluate_compiled(c, inputs)
    scale = max(1.0, max_abs(cpu[0]))
    assert_close(gpu[0], cpu[0], 1e-5, 1e-5 * scale, f"{name} {passes}")
    # Unoptimised CPU graph vs optimised GPU graph: pins the passes too.
    if passes == "default":
        ref = mc.Compiled(path=mc.graph_path(name), dims=dims, passes="none", backend="none")
        cpu0 = oracle.evaluate_compiled(ref, inputs)
        assert_close(gpu[0], cpu0[0], 1e-5, 1e-5 * max(1.0, max_abs(cpu0[0])), f"{name} vs unoptimised")


@pytest.mark.parametrize("first", [1, 51, 101, 151])
def test_random_graphs_match_the_cpu_oracle(device, mc, oracle, first):
    # tests/test_cuda_backend.cpp:418-437: seeds 1..200 (here in four runs of
    # 50), 1e-4 of each output's magnitude.
    seeds = list(range(first, first + 50))
    print(f"case random graphs seeds {first}..{first + 49}", flush=True)

    def build(seed):
        text = make_random_graph(seed, 24)
        return seed, [(p, mc.Compiled(text, passes=p)) for p in ("none", "default")]

    # hipRTC builds outside the kernel cache's lock; 16 threads, the GPU box's CPU share.
    with futures.ThreadPoolExecutor(max_workers=16) as pool:
        compiled = list(pool.map(build, seeds))
    for seed, pairs in compiled:
        for passes, c in pairs:
            inputs = uniform_inputs(oracle, c.input_sizes, seed)
            gpu = c.run(inputs)
            cpu = oracle.evaluate_compiled(c, inputs)
            assert len(gpu) == len(cpu)
            for k in range(len(cpu)):
                assert_close(gpu[k], cpu[k], 1e-4, 1e-4 * max(1.0, max_abs(cpu[k])), f"seed {seed} {passes} out {k}")
            c.close()


def test_fusion_cuts_kernel_launches(device, mc):
    # tests/test_cuda_backend.cpp:439-451, from tests/golden/reference_known_answers.json.
    import json
    from pathlib import Path
    case = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())["launch_counts"]

    def launches(passes):
        return mc.Compiled(path=mc.graph_path(case["graph"]), dims=case["dims"], passes=passes).kernel_launches
    for passes in ("none", "dne,fold,dne", "default"):
        assert launches(passes) == case[passes], passes


def test_reuses_intermediate_buffers_on_the_device(device, mc):
    text = "input x : f32[1024]\n" + "".join(f"v{i+1} = tanh {'x' if i == 0 else f'v{i}'}\n" for i in range(8))
    # tests/test_cuda_backend.cpp:453-461 compiles the unoptimised chain.
    c = mc.Compiled(text + "output v8\n", passes="none")
    assert c.kernel_launches == 8
    assert c.intermediate_bytes == 2 * 4096


def test_runs_repeatedly_on_device_resident_inputs(device, mc, oracle):
    # tests/test_cuda_backend.cpp:449-468.
    c = mc.Compiled(make_random_graph(17))
    inputs = uniform_inputs(oracle, c.input_sizes, 2)
    expected = c.run(inputs)
    c.upload(inputs)
    c.enqueue()
    c.enqueue()
    got = c.download()
    for e, g in zip(expected, got):
        assert np.array_equal(e, g)


def test_rejects_mismatched_inputs(device, mc):
    c = mc.Compiled(unary_graph("exp", (4,)))
    with pytest.raises(ValueError):
        c.run([])
    with pytest.raises(ValueError):
        c.run([np.zeros(5, np.float32)])
    assert c.run([np.zeros(4, np.float32)])[0].tolist() == [1.0] * 4


def test_outputs_are_written_in_place_into_bound_device_memory(device, mc, oracle):
    c = mc.Compiled(path=mc.graph_path("mlp_gelu"), dims={"B": 64, "D": 64, "H": 256})
    inputs = uniform_inputs(oracle, c.input_sizes, 4)
    expected = c.run(inputs)[0]
    x = mc.DeviceBuffer.from_array(inputs[0])
    y = mc.DeviceBuffer(expected.nbytes)
    y.fill_bytes(0xFF)
    c.bind_inputs([x.ptr])
    c.bind_outputs([y.ptr])
    assert c.output_ptr(0) == y.ptr and c.input_ptr(0) == x.ptr
    c.enqueue()
    c.synchronize()
    assert np.array_equal(y.download(), expected)
    # A graph output that is an input is copied into the bound buffer.
    c2 = mc.Compiled("input x : f32[8]\ny = neg x\noutput x, y\n")
    a = mc.DeviceBuffer.from_array(np.arange(8, dtype=np.float32))
    o0, o1 = mc.DeviceBuffer(32), mc.DeviceBuffer(32)
    c2.bind_inputs([a.ptr])
    c2.bind_outputs([o0.ptr, o1.ptr])
    c2.enqueue()
    c2.synchronize()
    assert o0.download().tolist() == list(range(8)) and o1.download().tolist() == [-float(i) for i in range(8)]


def test_the_pre_cast_matrix_core_path_matches_the_staging_path(device, mc, oracle):
    m, k, n = 256, 512, 384
    a = oracle.uniform(m * k, 1, -1, 1)
    b = oracle.uniform(k * n, 2, -1, 1)
    da, db = mc.DeviceBuffer.from_array(a), mc.DeviceBuffer.from_array(b)
    for kernel, dtype in (("tensor_core_bf16", mc.DTYPE_BF16), ("tensor_core_f16", mc.DTYPE_F16)):
        ha, hb = mc.DeviceBuffer(m * k * 2), mc.DeviceBuffer(k * n * 2)
        mc.convert_f32(dtype, da.ptr, ha.ptr, m * k)
        mc.convert_f32(dtype, db.ptr, hb.ptr, k * n)
        c1, c2 = mc.DeviceBuffer(m * n * 4), mc.DeviceBuffer(m * n * 4)
        mc.launch_matmul(kernel, da.ptr, db.ptr, c1.ptr, m, n, k)
        mc.launch_matmul_lowp(kernel, dtype, ha.ptr, hb.ptr, c2.ptr, m, n, k)
        mc.synchronize()
        assert np.array_equal(c1.download(), c2.download()), kernel
        # The device conversion is the oracle's rounding, bit for bit.
        rnd = oracle.round_bf16(a) if dtype == mc.DTYPE_BF16 else oracle.round_f16(a)
        bits = ha.download(np.uint16).astype(np.uint32)
        if dtype == mc.DTYPE_BF16:
            assert np.array_equal((bits << 16).view(np.float32), rnd)
        else:
            assert np.array_equal(bits.astype(np.uint16).view(np.float16).astype(np.float32), rnd)


MLP = ("mlp_gelu", {"B": 256}), ("mlp_gelu", {"B": 1024})


@pytest.mark.parametrize("name,dims", MLP + (("matmul_bias_gelu", {"M": 300, "K": 256, "N": 520}),
                                             ("matmul_bias_relu", None)))
@pytest.mark.parametrize("matmul", ["auto", "double_buffered", "split_k"])
def test_fused_gemm_epilogues_equal_the_separate_kernels_bit_for_bit(device, mc, oracle, name, dims, matmul):
    # The GEMM's store applies the consuming elementwise group: the same fp32
    # accumulation and the same per-op rounding, so identical bits.
    fused = mc.Compiled(path=mc.graph_path(name), dims=dims, options={"matmul": matmul})
    apart = mc.Compiled(path=mc.graph_path(name), dims=dims, options={"matmul": matmul, "epilogue": 0})
    assert any(len(ids) > 1 for ids in fused.launch_nodes), fused.launch_names
    if name == "mlp_gelu":
        # Both GEMMs carry their group: bias+GELU, and b2 + residual (whose
        # planned buffer is GEMM2's input, so its output is placed apart).
        assert fused.kernel_launches == 2, fused.launch_names
    assert all(len(ids) == 1 for ids in apart.launch_nodes)
    assert fused.kernel_launches < apart.kernel_launches
    inputs = uniform_inputs(oracle, fused.input_sizes, 1)
    a, b = fused.run(inputs), apart.run(inputs)
    for x, y in zip(a, b):
        assert np.array_equal(x.view(np.uint32), y.view(np.uint32)), (name, matmul)
    cpu = oracle.evaluate_compiled(fused, inputs)
    assert_close(a[0], cpu[0], 1e-4, 1e-4 * max(1.0, max_abs(cpu[0])), f"{name} fused vs CPU")


def test_epilogue_fusion_is_refused_when_the_group_is_not_next_or_reads_the_product_twice(device, mc, oracle):
    # A compute node between the matmul and its consumer: not fused (the
    # consumer's other input is computed after the matmul).
    text = """input a : f32[64, 32]
input w : f32[32, 48]
input z : f32[64, 48]
h = matmul a, w
e = exp z
s = add h, e
t = mul s, s
output t
"""
    c = mc.Compiled(text)
    inputs = uniform_inputs(oracle, c.input_sizes, 3)
    gpu = c.run(inputs)
    cpu = oracle.evaluate_compiled(c, inputs)
    assert_close(gpu[0], cpu[0], 1e-4, 1e-4 * max(1.0, max_abs(cpu[0])))
    graph = c.graph()
    matmul_ids = [n["id"] for n in graph["nodes"] if n["op_name"] == "matmul"]
    for ids in c.launch_nodes:
        if ids[0] in matmul_ids:
            # fused only if the consumer is the very next compute node
            assert len(ids) == 1 or ids[1] == ids[0] + 1
    # The product also a graph output: never fused.
    text2 = "input a : f32[64, 32]\ninput w : f32[32, 48]\nh = matmul a, w\ny = relu h\noutput h\noutput y\n"
    c2 = mc.Compiled(text2)
    assert all(len(ids) == 1 for ids in c2.launch_nodes)
    inputs2 = uniform_inputs(oracle, c2.input_sizes, 4)
    for g, r in zip(c2.run(inputs2), oracle.evaluate_compiled(c2, inputs2)):
        assert_close(g, r, 1e-4, 1e-4 * max(1.0, max_abs(r)))
