"""The elementwise kernel generator, without a GPU: the reference's generator
known answers (tests/test_cuda_codegen.cpp:29-109) restated for the HIP
text, and hipRTC compiling the generated kernels for gfx950 offline."""

import re

import pytest

GELU = """input x : f32[8, 64]
const coef : f32[] = 0.044715
const c : f32[] = 0.7978846
const half : f32[] = 0.5
const one : f32[] = 1.0
x2 = mul x, x
x3 = mul x2, x
t = mul x3, coef
inner = add x, t
u = mul inner, c
th = tanh u
hx = mul x, half
p = add th, one
y = mul hx, p
output y
"""


def kernel_loop(src):
    return src.index("for (; i +")


def test_fused_gelu_is_one_vectorised_kernel(mc):
    c = mc.Compiled(GELU, passes="fuse", backend="none")
    (src,) = c.kernel_sources
    assert "mc_elementwise(float* __restrict__ out, const float* __restrict__ in0, unsigned n)" in src
    assert "16-byte vector accesses" in src
    assert "reinterpret_cast<const mc_f32x4*>(in0)[p]" in src
    # Exact bit patterns, once, in the program (before the kernel's loop).
    assert src.count("__uint_as_float(0x3f000000u)") == 1
    assert src.index("0x3f000000u") < kernel_loop(src)
    # (x / 2)(1 + tanh u) is x times one mc_half_one_plus_tanh, x + x^3 coef one fmaf, in the program ...
    assert "r0 * mc_half_one_plus_tanh(r7)" in src and "mc_tanh" not in src and "mc_one_plus_tanh" not in src
    assert src.count("float mc_half_one_plus_tanh(float x)") == 1  # (defined once)
    assert src.count("fmaf(") == 1
    assert src.count("mc_program(a0[u].") == 8     # ... applied to 4 lanes, full and ragged steps


def program_of(src):
    return src[src.index("float mc_program("):src.index("extern")]


def test_multi_op_programs_contract_a_mul_used_once_into_its_add_or_sub(mc):
    shapes = [(64,), (64,), (64,)]
    # x y + z, z - x y, x y - z: one fmaf each, the mul not emitted alone.
    for text, call in (("r3 = mul r0, r1\nr4 = add r3, r2\n", "fmaf(r0, r1, r2)"),
                       ("r3 = mul r0, r1\nr4 = sub r2, r3\n", "fmaf(-r0, r1, r2)"),
                       ("r3 = mul r0, r1\nr4 = sub r3, r2\n", "fmaf(r0, r1, -r2)")):
        src, _ = mc.generate_elementwise_kernel("r0 = load in0\nr1 = load in1\nr2 = load in2\n" + text, shapes, (64,))
        body = program_of(src)
        assert f"const float r4 = {call};" in body and "const float r3" not in body, body
    # A mul with a second use stays a mul (and its add an add); a single op is never rewritten.
    src, _ = mc.generate_elementwise_kernel(
        "r0 = load in0\nr1 = load in1\nr2 = load in2\nr3 = mul r0, r1\nr4 = add r3, r2\nr5 = mul r4, r3\n", shapes, (64,))
    assert "fmaf" not in program_of(src)
    src, _ = mc.generate_elementwise_kernel("r0 = load in0\nr1 = load in1\nr2 = mul r0, r1\n", shapes[:2], (64,))
    assert "fmaf" not in program_of(src) and "const float r2 = r0 * r1;" in src
    # 1 + tanh u alone (not halved), or halved by a product used twice: mc_one_plus_tanh, the multiplies kept.
    src, _ = mc.generate_elementwise_kernel("r0 = load in0\nr1 = imm 1.0\nr2 = tanh r0\nr3 = add r2, r1\n"
                                            "r4 = mul r0, r3\n", shapes[:1], (64,))
    assert "const float r3 = mc_one_plus_tanh(r0);" in program_of(src) and "mc_half" not in src
    src, _ = mc.generate_elementwise_kernel("r0 = load in0\nr1 = imm 1.0\nr2 = tanh r0\nr3 = add r2, r1\n"
                                            "r4 = imm 0.5\nr5 = mul r0, r4\nr6 = mul r5, r3\nr7 = div r6, r5\n",
                                            shapes[:1], (64,))
    assert "mc_half" not in src and "const float r6 = r5 * r3;" in program_of(src)
    # tanh plus an immediate other than 1, or a tanh used twice: the plain tanh.
    src, _ = mc.generate_elementwise_kernel("r0 = load in0\nr1 = imm 2.0\nr2 = tanh r0\nr3 = add r2, r1\n",
                                            shapes[:1], (64,))
    assert "mc_one_plus_tanh" not in src and "mc_tanh(r0)" in src


def test_reads_a_bias_row_periodically(mc):
    add = "r0 = load in0\nr1 = load in1\nr2 = add r0, r1\n"
    src, vec = mc.generate_elementwise_kernel(add, [(16, 64), (64,)], (16, 64))
    assert vec and "[(p) % 16u]" in src
    src, vec = mc.generate_elementwise_kernel(add, [(16, 64), (64,)], (16, 64), allow_vectorize=False)
    assert not vec and "in1[(p) % 64u]" in src
    # A period that is not a multiple of 4 would let a vector straddle two repetitions.
    src, vec = mc.generate_elementwise_kernel(add, [(16, 6), (6,)], (16, 6))
    assert not vec and "in1[(p) % 6u]" in src


def test_general_broadcasts_use_constant_index_math(mc):
    mul = "r0 = load in0\nr1 = load in1\nr2 = mul r0, r1\n"
    src, vec = mc.generate_elementwise_kernel(mul, [(5, 4, 6), (5, 1, 6)], (5, 4, 6))
    assert not vec
    assert "in0[p]" in src
    assert "return (i / 24u) * 6u + (i % 6u);" in src and "in1[mc_general_1(p)]" in src
    src, _ = mc.generate_elementwise_kernel(mul, [(7, 9), (7, 1)], (7, 9))
    assert "return (i / 9u);" in src


def test_scalar_inputs_are_loaded_once_before_the_loop(mc):
    div = "r0 = load in0\nr1 = load in1\nr2 = div r0, r1\n"
    src, vec = mc.generate_elementwise_kernel(div, [(1000,), ()], (1000,))
    assert "const float s1 = in1[0];" in src and src.index("const float s1 = in1[0];") < kernel_loop(src)
    assert "const float r2 = r0 / r1;" in src
    assert vec  # 1000 is a multiple of 4
    _, vec = mc.generate_elementwise_kernel(div, [(1001,), ()], (1001,))
    assert not vec


def test_immediates_are_exact_bit_patterns(mc):
    prog = "r0 = load in0\nr1 = imm 0xbdcccccd\nr2 = mul r0, r1\nr3 = imm 0x7f800000\nr4 = add r2, r3\n"
    src, _ = mc.generate_elementwise_kernel(prog, [(8,)], (8,))
    assert "__uint_as_float(0xbdcccccdu)" in src  # -0.1f
    assert "__uint_as_float(0x7f800000u)" in src  # +inf
    src, _ = mc.generate_elementwise_kernel("r0 = load in0\nr1 = imm -0.1\nr2 = mul r0, r1\n", [(8,)], (8,))
    assert "__uint_as_float(0xbdcccccdu)" in src


UNARY = ["neg", "exp", "log", "sqrt", "relu", "sigmoid", "tanh"]
BINARY = ["add", "sub", "mul", "div"]


def test_every_op_is_emitted(mc):
    for op in UNARY:
        src, _ = mc.generate_elementwise_kernel(f"r0 = load in0\nr1 = {op} r0\n", [(4,)], (4,))
        assert "not an elementwise op" not in src
    for op in BINARY:
        src, _ = mc.generate_elementwise_kernel(f"r0 = load in0\nr1 = load in1\nr2 = {op} r0, r1\n", [(4,), (4,)], (4,))
        assert "not an elementwise op" not in src


def test_items_per_lane_controls_the_unroll(mc):
    src, _ = mc.generate_elementwise_kernel("r0 = load in0\nr1 = neg r0\n", [(4096,)], (4096,), items_per_lane=2)
    assert "for (; i + 256u < n; i += step)" in src and "gridDim.x * 512u" in src


def test_rejects_malformed_programs(mc):
    with pytest.raises(mc.MinicompilerError):
        mc.generate_elementwise_kernel("r0 = load in3\n", [(4,)], (4,))
    with pytest.raises(mc.MinicompilerError):
        mc.generate_elementwise_kernel("r0 = load in0\nr1 = add r0, r5\n", [(4,)], (4,))


@pytest.mark.parametrize("text,shapes,out", [
    (GELU, None, None),
    ("r0 = load in0\nr1 = load in1\nr2 = sub r0, r1\nr3 = load in2\nr4 = div r2, r3\nr5 = relu r4\n",
     [(64, 256), (256,), (256,)], (64, 256)),
    ("r0 = load in0\nr1 = load in1\nr2 = mul r0, r1\nr3 = sigmoid r2\nr4 = log r3\nr5 = exp r4\nr6 = sqrt r5\n",
     [(5, 4, 6), (5, 1, 6)], (5, 4, 6)),
    ("r0 = load in0\nr1 = load in1\nr2 = add r0, r1\n", [(17, 1), (1, 33)], (17, 33)),
])
def test_generated_kernels_compile_for_gfx950_without_a_gpu(mc, text, shapes, out):
    if shapes is None:
        src = mc.Compiled(text, passes="fuse", backend="none").kernel_sources[0]
    else:
        src, _ = mc.generate_elementwise_kernel(text, shapes, out)
    ok, log = mc.compile_kernel_source(src, "gfx950")
    assert ok, log


@pytest.mark.parametrize("body,call", [("ring_big", "mc_gemm_f32_ring<McRingBig>"),
                                       ("ring_wide", "mc_gemm_f32_ring<McRingWide>"),
                                       ("ring_wide8", "mc_gemm_f32_ring<McRingWide8>"),
                                       ("ring_thin", "mc_gemm_f32_ring<McRingThin>"),
                                       ("ring_mid", "mc_gemm_f32_ring<McRingMid>"),
                                       ("narrow16", "mc_gemm_f32_narrow<McNarrow16>"),
                                       ("narrow32", "mc_gemm_f32_narrow<McNarrow32>"),
                                       ("narrow16x64", "mc_gemm_f32_narrow<McNarrow16x64>"),
                                       ("narrow16x32", "mc_gemm_f32_narrow<McNarrow16x32>"),
                                       ("bf16", "mc_gemm16_fast<true, true>"), ("f16", "mc_gemm16_fast<false, true>")])
def test_every_gemm_body_with_an_epilogue_compiles_for_gfx950(mc, body, call):
    # bias + tanh on the product, as a fused group reads it: each GEMM body the
    # executable can pick, compiled by hipRTC with no device.
    text = "r0 = load in0\nr1 = load in1\nr2 = add r0, r1\nr3 = tanh r2\n"
    src = mc.generate_gemm_epilogue_kernel(text, 0, [(96, 256), (256,)], (96, 256), True, body)
    assert call in src
    ok, log = mc.compile_kernel_source(src, "gfx950")
    assert ok, log
    with pytest.raises(mc.MinicompilerError, match="unknown body"):
        mc.generate_gemm_epilogue_kernel(text, 0, [(96, 256), (256,)], (96, 256), True, "tiny")


def test_a_bad_generated_source_returns_the_hiprtc_log(mc):
    ok, log = mc.compile_kernel_source('extern "C" __global__ void mc_elementwise() { undefined_thing(); }')
    assert not ok and "undefined_thing" in log and "hipRTC could not compile" in log


@pytest.mark.parametrize("text,acc,shapes,out,vec", [
    # bias + GELU on a GEMM result (the MLP's first group), 16-byte operand loads
    (GELU.replace("load in0", "load in0"), 0, None, None, True),
    # bias + residual, the product as the second input; scalar operand loads
    ("r0 = load in0\nr1 = load in1\nr2 = add r0, r1\nr3 = load in2\nr4 = add r2, r3\n", 1,
     [(512,), (64, 512), (64, 512)], (64, 512), False),
    # a general broadcast and a scalar next to the product
    ("r0 = load in0\nr1 = load in1\nr2 = mul r0, r1\nr3 = load in2\nr4 = sub r2, r3\n", 0,
     [(5, 8), (5, 1), ()], (5, 8), True),
])
def test_gemm_epilogue_kernels_compile_for_gfx950_without_a_gpu(mc, text, acc, shapes, out, vec):
    if shapes is None:
        shapes, out = [(64, 128)], (64, 128)
        text = "r0 = load in0\nr1 = imm 0x3f000000\nr2 = mul r0, r1\nr3 = tanh r2\n"
    src = mc.generate_gemm_epilogue_kernel(text, acc, shapes, out, vec)
    assert "mc_gemm_f32_mfma<true, " + ("true" if vec else "false") + ">" in src
    assert "extern \"C\" __global__ void __launch_bounds__(256, 2)\nmc_gemm_epilogue(" in src
    assert "mc_sum_splits_epilogue(" in src
    # The product enters the program as the accumulated value, the others by access class.
    call = src[src.index("return mc_program("):].split("\n")[0]
    assert call.split("(", 1)[1].split(",")[acc].strip(" );") == "v"
    ok, log = mc.compile_kernel_source(src, "gfx950")
    assert ok, log
