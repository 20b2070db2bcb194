"""Pins the CPU oracle before anything is checked against it.

Each oracle function is checked against something that does not share its
code: the reference's golden bits, closed forms, numpy's own IEEE float32
arithmetic and broadcasting, Python's math library, the double-precision
evaluator, and the reference's known answers.
"""

import math
import struct

import numpy as np
import pytest

from helpers import all_close, assert_close, gamma, U32

UNARY = ["neg", "exp", "log", "sqrt", "relu", "sigmoid", "tanh"]
BINARY = ["add", "sub", "mul", "div"]
PATTERNS = [((17, 33), (17, 33)), ((17, 32), ()), ((), (17, 33)), ((17, 32), (32,)), ((17, 33), (17, 1)),
            ((17, 1), (1, 33)), ((2, 3, 4), (3, 1)), ((5, 1, 6), (1, 4, 1))]


def bits(x: float) -> int:
    return struct.unpack("<I", struct.pack("<f", x))[0]


def test_uniform_matches_the_reference_golden_bits(oracle):
    # tests/test_parser.cpp:136-147: uniform_values(4, 42, -0.3f, 0.7f).
    v = oracle.uniform(4, 42, -0.3, 0.7)
    assert [bits(float(x)) for x in v] == [0x3EE214CA, 0xBE0F73A8, 0xBCAF4CC0, 0x3D350140]


def splitmix_numpy(count: int, seed: int, lo: float, hi: float) -> np.ndarray:
    """An independent numpy statement of the generator (uint64 wraparound)."""
    with np.errstate(over="ignore"):
        idx = np.arange(1, count + 1, dtype=np.uint64)
        z = np.uint64(seed) + idx * np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        z = z ^ (z >> np.uint64(31))
    u = (z >> np.uint64(40)).astype(np.float32) * np.float32(2.0 ** -24)
    lo32, hi32 = np.float32(lo), np.float32(hi)
    return lo32 + (hi32 - lo32) * u  # float32 ops, each rounded


def test_uniform_matches_an_independent_numpy_generator(oracle):
    for seed, lo, hi in [(1, -3.0, 3.0), (123, -2.0, 3.0), (7, 0.5, 2.0)]:
        a = oracle.uniform(10000, seed, lo, hi)
        b = splitmix_numpy(10000, seed, lo, hi)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        assert a.min() >= np.float32(lo) and a.max() < np.float32(hi)


def test_normal_has_the_requested_moments_and_is_deterministic(oracle):
    z = oracle.normal(1 << 20, 1, 0.0, 1.0).astype(np.float64)
    assert abs(z.mean()) < 4e-3 and abs(z.std() - 1.0) < 4e-3
    # Box-Muller pairs: z0^2 + z1^2 = -2 ln u1 > 0, so no pair is (0, 0).
    assert np.array_equal(oracle.normal(101, 9, 0.5, 0.1), oracle.normal(101, 9, 0.5, 0.1))
    small = oracle.normal(1000, 2, 0.0, 0.1).astype(np.float64)
    assert abs(small.std() - 0.1) < 0.01


@pytest.mark.parametrize("op", UNARY)
def test_unary_ops_match_the_double_evaluator(oracle, op):
    # tests/test_cpu_backend.cpp:55-79: exact for neg/relu, 2.4e-7 rel for
    # sqrt, rtol 1e-6 + atol 1.2e-7 for the transcendental functions.
    lo = 0.01 if op in ("log", "sqrt") else -6.0
    x = oracle.uniform(37 * 29, 11, lo, 6.0)
    got = oracle.unary(op, x)
    ref = oracle.unary(op, x, reference=True)
    rtol, atol = (0.0, 0.0) if op in ("neg", "relu") else ((2.4e-7, 0.0) if op == "sqrt" else (1e-6, 1.2e-7))
    assert_close(got, ref, rtol, atol, op)


def test_unary_closed_forms(oracle):
    x = np.array([0.0, 1.0, 4.0, -2.5, 0.25], dtype=np.float32)
    assert oracle.unary("exp", x[:1])[0] == 1.0
    assert oracle.unary("log", x[1:2])[0] == 0.0
    assert oracle.unary("sqrt", x[2:3])[0] == 2.0
    assert oracle.unary("tanh", x[:1])[0] == 0.0
    assert oracle.unary("sigmoid", x[:1])[0] == 0.5
    assert list(oracle.unary("relu", x)) == [0.0, 1.0, 4.0, 0.0, 0.25]
    assert list(oracle.unary("neg", x)) == [-0.0, -1.0, -4.0, 2.5, -0.25]
    for v in (-3.0, -0.7, 0.3, 2.0):
        a = np.array([v], dtype=np.float32)
        for op, f in (("exp", math.exp), ("tanh", math.tanh), ("sigmoid", lambda t: 1 / (1 + math.exp(-t)))):
            assert abs(float(oracle.unary(op, a)[0]) - f(float(a[0]))) <= 4 * U32 * abs(f(float(a[0]))) + 1e-12


@pytest.mark.parametrize("sa,sb", PATTERNS)
def test_binary_broadcasting_matches_numpy_bit_for_bit(oracle, sa, sb):
    # numpy's float32 + - * / are IEEE and its broadcasting is an
    # independent implementation of the same rule.
    a = oracle.uniform(int(np.prod(sa, dtype=np.int64)), 5, 0.5, 2.0)
    b = oracle.uniform(int(np.prod(sb, dtype=np.int64)), 6, 0.5, 2.0)
    out = np.broadcast_shapes(sa, sb)
    fns = {"add": np.add, "sub": np.subtract, "mul": np.multiply, "div": np.divide}
    for op in BINARY:
        expect = fns[op](a.reshape(sa), b.reshape(sb)).astype(np.float32).reshape(-1)
        for reference in (False, True):
            got = oracle.binary(op, a, sa, b, sb, out, reference=reference)
            assert np.array_equal(got.view(np.uint32), expect.view(np.uint32)), (op, sa, sb, reference)


def fused_every_load_kind():
    # out = tanh(x * s + row) - col / 2 over [37, 41]: x contiguous, s a
    # scalar, row periodic, col general (tests/test_cpu_backend.cpp:133-155).
    program = [
        {"kind": 0, "op": 0, "a": 0, "b": -1, "imm_bits": 0},   # r0 = x
        {"kind": 0, "op": 0, "a": 1, "b": -1, "imm_bits": 0},   # r1 = s
        {"kind": 3, "op": 11, "a": 0, "b": 1, "imm_bits": 0},   # r2 = x * s
        {"kind": 0, "op": 0, "a": 2, "b": -1, "imm_bits": 0},   # r3 = row
        {"kind": 3, "op": 9, "a": 2, "b": 3, "imm_bits": 0},    # r4 = r2 + row
        {"kind": 2, "op": 8, "a": 4, "b": -1, "imm_bits": 0},   # r5 = tanh
        {"kind": 0, "op": 0, "a": 3, "b": -1, "imm_bits": 0},   # r6 = col
        {"kind": 1, "op": 1, "a": -1, "b": -1, "imm_bits": bits(2.0)},  # r7 = 2
        {"kind": 3, "op": 12, "a": 6, "b": 7, "imm_bits": 0},   # r8 = col / 2
        {"kind": 3, "op": 10, "a": 5, "b": 8, "imm_bits": 0},   # r9 = r5 - r8
    ]
    shapes = [(37, 41), (), (41,), (37, 1)]
    return program, shapes, (37, 41)


def test_fused_program_every_load_kind(oracle):
    program, shapes, out = fused_every_load_kind()
    ins = [oracle.uniform(int(np.prod(s, dtype=np.int64)), 20 + i, -1.0, 1.0) for i, s in enumerate(shapes)]
    got = oracle.fused(program, ins, shapes, out)
    ref = oracle.fused(program, ins, shapes, out, reference=True)
    assert_close(got, ref, 1e-6, 1.2e-7, "cpu vs double")
    # numpy, float32 per op, with its own broadcasting; tanh from numpy (a
    # different implementation), hence the tolerance.
    x, s, row, col = (ins[0].reshape(37, 41), np.float32(ins[1][0]), ins[2], ins[3].reshape(37, 1))
    expect = (np.tanh((x * s) + row) - col / np.float32(2.0)).astype(np.float32).reshape(-1)
    assert_close(got, expect, 1e-6, 1.2e-7, "cpu vs numpy")
    # 1517 elements: the last 512-element block is partial; threads do not change the result.
    oracle.set_threads(4)
    try:
        assert np.array_equal(oracle.fused(program, ins, shapes, out), got)
    finally:
        oracle.set_threads(1)


def test_fused_program_with_scalar_only_registers_fills_the_output(oracle):
    # A program whose result never touches a vector input (an immediate
    # chain) is a constant fill (src/cpu/kernels.cpp:254-261).
    program = [{"kind": 0, "op": 0, "a": 0, "b": -1, "imm_bits": 0},
               {"kind": 1, "op": 1, "a": -1, "b": -1, "imm_bits": bits(3.0)},
               {"kind": 2, "op": 2, "a": 1, "b": -1, "imm_bits": 0}]
    x = oracle.uniform(600, 1, -1, 1)
    assert np.all(oracle.fused(program, [x], [(600,)], (600,)) == -3.0)


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (3, 5, 7), (64, 64, 64), (33, 257, 65), (130, 300, 70)])
def test_matmul_is_within_the_dot_product_bound(oracle, m, k, n):
    # tests/test_cpu_backend.cpp:81-110: within gamma_k sum|ab| + u|e| of
    # the exact (double) product rounded to float.
    a = oracle.uniform(m * k, 3, -1, 1)
    b = oracle.uniform(k * n, 4, -1, 1)
    c = oracle.matmul(a, b, m, k, n)
    exact, absdot = oracle.gemm_f64(a, b, m, k, n)
    e = exact.astype(np.float32).astype(np.float64)
    assert np.all(np.abs(c - e) <= gamma(k) * absdot + U32 * np.abs(e))
    # The double evaluator is the exact product rounded once.
    assert np.array_equal(oracle.matmul(a, b, m, k, n, reference=True), exact.astype(np.float32))
    # numpy's float64 GEMM agrees with the oracle's float64 dot products.
    np.testing.assert_allclose(exact, (a.reshape(m, k).astype(np.float64) @ b.reshape(k, n).astype(np.float64)).reshape(-1),
                               rtol=1e-12, atol=1e-12)


def test_matmul_threads_do_not_change_results(oracle):
    a = oracle.uniform(37 * 64, 1, -1, 1)
    b = oracle.uniform(64 * 50, 2, -1, 1)
    one = oracle.matmul(a, b, 37, 64, 50)
    oracle.set_threads(5)
    try:
        assert np.array_equal(oracle.matmul(a, b, 37, 64, 50), one)
    finally:
        oracle.set_threads(1)


def test_bf16_and_f16_rounding_known_answers(oracle):
    one = 1.0
    x = np.array([one, one + 2 ** -8, one + 3 * 2 ** -8, -one - 2 ** -8, 3.4028234663852886e38, np.inf, 1e-40],
                 dtype=np.float32)
    r = oracle.round_bf16(x)
    assert r[0] == 1.0
    assert r[1] == 1.0                      # halfway: ties to even (mantissa 0)
    assert r[2] == one + 2 ** -6            # halfway between odd and even: up to even
    assert r[3] == -1.0
    assert np.isinf(r[4]) and r[4] > 0      # above the last halfway point: overflows
    assert np.isinf(r[5])
    # subnormal 1e-40 = 0x000116c2: the low half 0x16c2 is below halfway -> 0x00010000
    assert np.float32(1e-40).view(np.uint32) == 0x000116C2
    assert r[6].view(np.uint32) == 0x00010000
    nan = oracle.round_bf16(np.array([np.nan], dtype=np.float32))
    assert np.isnan(nan[0])
    # fp16: spacing at 1 is 2^-10.
    h = oracle.round_f16(np.array([1 + 2 ** -11, 1 + 3 * 2 ** -11, 65520.0, 2 ** -25], dtype=np.float32))
    assert h[0] == 1.0 and h[1] == 1 + 2 ** -9 and np.isinf(h[2]) and h[3] == 0.0


def test_random_graphs_match_the_double_precision_evaluator(mc, oracle):
    # CpuBackend.RandomGraphsMatchReference (tests/test_cpu_backend.cpp:176-191):
    # the fp32 restatement against the float64 evaluator (every node rounded
    # to float) on 200 unoptimised random graphs, 1e-4 of each output's
    # largest magnitude.
    from graphgen import make_random_graph

    for seed in range(1, 201):
        c = mc.Compiled(make_random_graph(seed), passes="none", backend="none")
        inputs = [oracle.uniform(n, seed + k, -1.0, 1.0) for k, n in enumerate(c.input_sizes)]
        actual = oracle.evaluate_compiled(c, inputs, mode="cpu")
        expected = oracle.evaluate_compiled(c, inputs, mode="reference")
        assert len(actual) == len(expected)
        for k, (a, e) in enumerate(zip(actual, expected)):
            scale = max(1.0, float(np.max(np.abs(e))) if e.size else 1.0)
            assert np.all(np.abs(a.astype(np.float64) - e) <= 1e-4 * np.abs(e) + 1e-4 * scale), (seed, k)
        c.close()
