"""The callers of the backend: parser, passes and memory planner, through the
C ABI with backend "none" (no device). Known answers are the reference's
(tests/test_end_to_end.cpp, test_operator_fusion.cpp, test_constant_folding.cpp,
test_memory_plan.cpp, test_parser.cpp); equivalence checks use the CPU oracle.
"""

import struct

import numpy as np
import pytest

from graphgen import make_random_graph
from helpers import assert_close, max_abs


def compile_none(mc, text, passes="default", dims=None):
    return mc.Compiled(text, passes=passes, dims=dims, backend="none")


def node_named(g, name):
    return next(n for n in g["nodes"] if n["name"] == name)


def f32_bits(v):
    return struct.unpack("<I", struct.pack("<f", v))[0]


def stage_counts(c):
    return [(s["stats"]["nodes"], s["stats"]["compute_nodes"]) for s in c.stage_stats()]


@pytest.mark.parametrize("name,dims,expected", [
    ("gelu_chain", {"M": 64, "N": 300}, [(17, 11), (17, 11), (17, 9), (14, 9), (6, 1), (2, 1)]),
    ("matmul_bias_relu", {"M": 33, "K": 70, "N": 129}, [(6, 3), (6, 3), (6, 3), (6, 3), (5, 2), (5, 2)]),
    ("mlp_block_bn", {"B": 16, "D": 64, "H": 256}, [(37, 22), (37, 22), (37, 18), (31, 18), (17, 4), (13, 4)]),
])
def test_stage_counts_match_the_reference(mc, name, dims, expected):
    # tests/test_end_to_end.cpp:86, 98, 112 (input, dne, fold, dne, fuse, dne).
    c = mc.Compiled(path=mc.graph_path(name), dims=dims, backend="none")
    assert stage_counts(c) == expected
    if name == "mlp_block_bn":
        s = c.stage_stats()[-1]["stats"]
        assert (s["matmuls"], s["fused_nodes"], s["elementwise_ops"]) == (2, 2, 16)
    if name == "gelu_chain":
        s = c.stage_stats()[-1]["stats"]
        assert (s["fused_nodes"], s["elementwise_ops"]) == (1, 9)


def test_gelu_fuses_into_one_program_with_one_load_and_four_immediates(mc):
    c = mc.Compiled(path=mc.graph_path("gelu_chain"), dims={"M": 8, "N": 64}, backend="none")
    g = c.graph()
    y = g["nodes"][g["outputs"][0]]
    assert y["op_name"] == "fused" and y["name"] == "y" and len(y["inputs"]) == 1
    prog = y["program"]
    assert sum(p["kind"] == 0 for p in prog) == 1
    imms = [p["imm_bits"] for p in prog if p["kind"] == 1]
    # coef, folded sqrt(2/pi), one, half in first-use order.
    sqrt_2_over_pi = np.sqrt(np.float32(2.0) / np.float32(3.14159265358979))
    assert imms == [f32_bits(0.044715), f32_bits(float(sqrt_2_over_pi)), f32_bits(1.0), f32_bits(0.5)]
    assert y["sources"] == ["x2", "x3", "t", "inner", "u", "th", "p", "hx", "y"]
    # The program's instruction order (loads/immediates at first use, operand a before b).
    kinds = [(p["kind"], p["op"], p["a"], p["b"]) for p in prog]
    assert kinds == [(0, 0, 0, -1), (3, 11, 0, 0), (3, 11, 1, 0), (1, 1, -1, -1), (3, 11, 2, 3), (3, 9, 0, 4),
                     (1, 1, -1, -1), (3, 11, 5, 6), (2, 8, 7, -1), (1, 1, -1, -1), (3, 9, 8, 9), (1, 1, -1, -1),
                     (3, 11, 0, 11), (3, 11, 12, 10)]


FUSION_CASES = {
    # test_operator_fusion.cpp:82-97: a matmul splits groups; a non-scalar constant is loaded.
    "matmul_splits": ("input x : f32[4, 8]\nconst w : f32[8, 16] = 0.1\nconst b : f32[16] = 0.2\n"
                      "h = matmul x, w\nhb = add h, b\ny = relu hb\noutput y\n", [["hb", "y"]]),
    # :99-110: a producer read outside the group stays out.
    "needed_outside": ("input x : f32[4, 4]\nconst w : f32[4, 4] = 1.0\na = exp x\nt = tanh a\ny = add t, x\n"
                       "z = matmul a, w\noutput y, z\n", [["t", "y"]]),
    # :112-118: a graph output is never fused away.
    "output": ("input x : f32[4]\na = exp x\nn = neg a\noutput a, n\n", []),
    # :120-131: a diamond fuses, the shared value computed once.
    "diamond": ("input x : f32[16]\na = tanh x\ne = exp a\nn = neg a\ny = add e, n\noutput y\n",
                [["a", "e", "n", "y"]]),
    # :133-141: a broadcast producer is not pulled in.
    "broadcast": ("input x : f32[4, 8]\ninput row : f32[8]\nv = exp row\ns = add x, v\ny = tanh s\noutput y\n",
                  [["s", "y"]]),
    # :143-156: no cycle through an outside node.
    "cycle": ("input x : f32[4, 4]\nconst w : f32[4, 4] = 0.5\na = exp x\nm = matmul a, w\ny = mul a, m\noutput y\n", []),
}


@pytest.mark.parametrize("case", sorted(FUSION_CASES))
def test_fusion_groups_match_the_reference(mc, case):
    text, groups = FUSION_CASES[case]
    c = compile_none(mc, text, passes="fuse")
    fused = [n for n in c.graph()["nodes"] if n["op_name"] == "fused"]
    assert [n["sources"] for n in fused] == groups
    if case == "diamond":
        assert sum(p["kind"] >= 2 for p in fused[0]["program"]) == 4
    if case == "matmul_splits":
        y = fused[0]
        g = c.graph()
        assert [g["nodes"][i]["op_name"] for i in y["inputs"]] == ["matmul", "const"]


def test_constant_folding_known_answers(mc):
    # test_constant_folding.cpp:31-72.
    text = ("input x : f32[4]\nconst two : f32[] = 2.0\nconst pi : f32[] = 3.14159265\n"
            "ratio = div two, pi\nc = sqrt ratio\ny = mul x, c\noutput y\n")
    c = compile_none(mc, text, passes="fold")
    g = c.graph()
    cn = node_named(g, "c")
    assert cn["op_name"] == "const"
    assert abs(float(c.constant(cn["id"])[0]) - np.sqrt(2.0 / 3.14159265)) <= 2e-7
    assert node_named(g, "ratio")["op_name"] == "const" and node_named(g, "y")["op_name"] == "mul"
    st = c.stage_stats()
    assert (st[0]["stats"]["compute_nodes"], st[1]["stats"]["compute_nodes"]) == (3, 1)

    bn = ("input x : f32[2, 3]\nconst var : f32[3] = [0.25, 1, 4]\nconst eps : f32[] = 0\n"
          "const gamma : f32[3] = [1, 2, 3]\nve = add var, eps\nsd = sqrt ve\nscale = div gamma, sd\n"
          "const w : f32[2, 3] = [1, 2, 3, 4, 5, 6]\nws = mul w, scale\nconst m : f32[2, 2] = [1, 2, 3, 4]\n"
          "sq = matmul m, ws\ny = add x, sq\noutput y\n")
    c = compile_none(mc, bn, passes="fold")
    g = c.graph()
    assert list(c.constant(node_named(g, "scale")["id"])) == [2.0, 2.0, 1.5]
    assert list(c.constant(node_named(g, "ws")["id"])) == [2, 4, 4.5, 8, 10, 9]
    assert list(c.constant(node_named(g, "sq")["id"])) == [18, 24, 22.5, 38, 52, 49.5]
    assert node_named(g, "y")["op_name"] == "add"


def test_folding_leaves_big_results_and_input_dependent_nodes(mc):
    # Folding caps results at 2^22 elements (constant_folding.hpp:11-15).
    text = ("input x : f32[2048, 2049]\nconst a : f32[2048, 2049] = 1.0\nconst b : f32[] = 2.0\n"
            "big = mul a, b\ny = add x, big\noutput y\n")
    g = compile_none(mc, text, passes="fold").graph()
    assert node_named(g, "big")["op_name"] == "mul"


PLAN_CASES = {
    # test_memory_plan.cpp:10-23: a chain ping-pongs between two buffers.
    "chain": "input x : f32[256]\nv1 = tanh x\nv2 = tanh v1\nv3 = tanh v2\nv4 = tanh v3\nv5 = tanh v4\nv6 = tanh v5\noutput v6\n",
    # :25-39
    "diamond": "input x : f32[8]\na = exp x\nn = neg a\nc = add a, n\noutput c\n",
    # :41-55
    "outputs": "input x : f32[8]\ny1 = exp x\nt = neg x\ny2 = tanh t\noutput y1, y2\n",
    # :88-99
    "dead": "input x : f32[8]\ndead = exp x\ny = neg x\noutput y\n",
    # :101-116
    "grow": "input v : f32[8]\ninput m : f32[4, 8]\na = exp v\nn = neg a\nc = add m, n\noutput c\n",
    # :72-86
    "chained_outputs": "input x : f32[64]\nh1 = exp x\ny1 = neg h1\nh2 = tanh y1\ny2 = neg h2\noutput y1, y2\n",
    # :57-70
    "caller_outputs": "input x : f32[8]\nt = exp x\ny = neg t\noutput y\n",
}


def plan_of(mc, case, pool=True):
    c = compile_none(mc, PLAN_CASES[case], passes="none")
    g = c.graph()
    ids = {n["name"]: n["id"] for n in g["nodes"]}
    return c.plan(pool), ids, g


def test_memory_plan_known_answers(mc):
    p, ids, g = plan_of(mc, "chain")
    assert len(p["buffer_bytes"]) == 2 and p["bytes_without_reuse"] == 6 * 1024 and p["bytes_with_reuse"] == 2048
    assert p["buffer_of"][ids["x"]] == -1

    p, ids, _ = plan_of(mc, "diamond")
    b = p["buffer_of"]
    assert p["last_use"][ids["a"]] == ids["c"]
    assert b[ids["a"]] != b[ids["n"]] and b[ids["c"]] not in (b[ids["a"]], b[ids["n"]])

    p, ids, g = plan_of(mc, "outputs")
    b = p["buffer_of"]
    assert p["last_use"][ids["y1"]] == len(g["nodes"])
    assert b[ids["y2"]] != b[ids["y1"]] and b[ids["t"]] != b[ids["y1"]]

    p, ids, _ = plan_of(mc, "dead")
    assert p["last_use"][ids["dead"]] == -1
    assert p["buffer_of"][ids["y"]] == p["buffer_of"][ids["dead"]] and len(p["buffer_bytes"]) == 1

    p, ids, _ = plan_of(mc, "grow")
    assert len(p["buffer_bytes"]) == 2 and p["buffer_of"][ids["c"]] == p["buffer_of"][ids["a"]]
    assert p["buffer_bytes"][p["buffer_of"][ids["c"]]] == 128

    p, ids, _ = plan_of(mc, "chained_outputs", pool=False)
    assert len(p["buffer_bytes"]) == 1 and p["buffer_of"][ids["h2"]] == p["buffer_of"][ids["h1"]]
    assert p["buffer_of"][ids["y1"]] == -1 and p["buffer_of"][ids["y2"]] == -1

    p, ids, _ = plan_of(mc, "caller_outputs", pool=False)
    assert p["buffer_of"][ids["y"]] == -1 and p["buffer_of"][ids["t"]] != -1 and p["bytes_without_reuse"] == 32


def test_shared_buffers_never_hold_two_live_values_on_random_graphs(mc):
    # test_memory_plan.cpp:125-146 (400 seeds, both output modes).
    for seed in range(1, 401):
        c = compile_none(mc, make_random_graph(seed // 2 + 1, 24), passes="none")
        g = c.graph()
        pool = seed % 2 == 0
        p = c.plan(pool)
        assert p["bytes_with_reuse"] <= p["bytes_without_reuse"]
        nodes = g["nodes"]
        for u in nodes:
            buf = p["buffer_of"][u["id"]]
            compute = u["op_name"] not in ("input", "const")
            if not compute or (not pool and u["id"] in g["outputs"]):
                assert buf == -1
                continue
            assert p["buffer_bytes"][buf] >= 4 * int(np.prod(u["shape"], dtype=np.int64))
            for v in nodes[u["id"] + 1:]:
                if p["buffer_of"][v["id"]] == buf:
                    assert p["last_use"][u["id"]] < v["id"], (seed, u["id"], v["id"])


def test_optimized_graphs_compute_what_unoptimized_ones_do(mc, oracle):
    # test_end_to_end.cpp:127-136 over the oracle: folding evaluates early,
    # fusion evaluates per element, nothing reassociates.
    removed = 0
    fused = 0
    for seed in range(1, 301):
        text = make_random_graph(seed, 24)
        ref = compile_none(mc, text, passes="none")
        opt = compile_none(mc, text, passes="default")
        removed += len(ref.graph()["nodes"]) - len(opt.graph()["nodes"])
        fused += opt.stage_stats()[-1]["stats"]["fused_nodes"]
        inputs = [oracle.uniform(n, seed + k, -1.0, 1.0) for k, n in enumerate(ref.input_sizes)]
        expected = oracle.evaluate_compiled(ref, inputs)
        actual = oracle.evaluate_compiled(opt, inputs)
        for k, (a, e) in enumerate(zip(actual, expected)):
            assert_close(a, e, 1e-5, 1e-5 * max(1.0, max_abs(e)), f"seed {seed} output {k}")
    assert removed > 1000 and fused > 150  # the reference's bound on removals: test_end_to_end.cpp:135


@pytest.mark.parametrize("name,dims", [("gelu_chain", {"M": 64, "N": 300}),
                                       ("matmul_bias_relu", {"M": 33, "K": 70, "N": 129}),
                                       ("mlp_block_bn", {"B": 16, "D": 64, "H": 256}),
                                       ("mlp_gelu", {"B": 16, "D": 64, "H": 256}),
                                       ("batchnorm_relu", {"R": 50}),
                                       ("matmul_bias_gelu", {"M": 20, "K": 30, "N": 40})])
def test_benchmark_graphs_optimized_equal_unoptimized(mc, oracle, name, dims):
    ref = mc.Compiled(path=mc.graph_path(name), dims=dims, passes="none", backend="none")
    opt = mc.Compiled(path=mc.graph_path(name), dims=dims, passes="default", backend="none")
    for seed in (1, 2, 3):
        inputs = [oracle.uniform(n, seed + k, -1.0, 1.0) for k, n in enumerate(ref.input_sizes)]
        e = oracle.evaluate_compiled(ref, inputs)[0]
        a = oracle.evaluate_compiled(opt, inputs)[0]
        assert_close(a, e, 1e-5, 1e-5 * max(1.0, max_abs(e)), name)


def test_every_benchmark_graph_parses_at_its_default_size(mc):
    for name in ("gelu_chain", "matmul_bias_relu", "mlp_block_bn", "mlp_gelu", "batchnorm_relu"):
        c = mc.Compiled(path=mc.graph_path(name), passes="none", backend="none")
        assert c.num_outputs == 1


def test_parser_errors_and_printer(mc):
    bad = {
        "input x : f32[2]\ny = frob x\noutput y\n": "unknown op 'frob'",
        "input x : f32[2]\ny = neg z\noutput y\n": "unknown value 'z'",
        "input x : f64[2]\noutput x\n": "only f32",
        "input x : f32[0]\noutput x\n": "invalid shape",
        "input x : f32[2]\ninput x : f32[2]\noutput x\n": "defined twice",
        "input x : f32[2]\n": "no outputs",
        "dim B = 4\ndim B = 5\ninput x : f32[B]\noutput x\n": "already declared",
        "input x : f32[65536, 65536]\noutput x\n": "2^31 - 1",
        "const c : f32[2] = uniform(seed=1, lo=2, hi=1)\noutput c\n": "lo must be below hi",
        "input x : f32[2, 3]\ninput y : f32[4]\nz = add x, y\noutput z\n": "cannot broadcast",
    }
    for text, needle in bad.items():
        with pytest.raises(mc.MinicompilerError) as e:
            compile_none(mc, text, passes="none")
        assert needle in str(e.value), (text, str(e.value))
    with pytest.raises(mc.MinicompilerError, match="declares no dim 'Q'"):
        compile_none(mc, "dim B = 4\ninput x : f32[B]\noutput x\n", dims={"Q": 2})
    with pytest.raises(mc.MinicompilerError, match="unknown pass"):
        compile_none(mc, "input x : f32[2]\noutput x\n", passes="dne,frob")
    # test_parser.cpp printer known answers.
    text = ("graph layer\ninput x : f32[2, 3]\nconst w : f32[3, 4] = 0.5\nconst b : f32[4] = [1, 2, 3, 4]\n"
            "h = matmul x, w\nhb = add h, b\nconst two : f32[] = 2\ny = mul hb, two\noutput y\n")
    p = compile_none(mc, text, passes="none").print_graph()
    assert "graph layer\n" in p
    assert "%0 x = input : f32[2,3]" in p
    assert "%2 b = const [1, 2, 3, 4] : f32[4]" in p
    assert "%6 y = mul %4, %5 : f32[2,4]  (output)" in p


def test_uniform_constants_carry_the_reference_golden_bits(mc):
    # The library's generator (src/random.cpp) through a parsed constant.
    c = compile_none(mc, "const v : f32[4] = uniform(seed=42, lo=-0.3, hi=0.7)\noutput v\n", passes="none")
    vals = c.constant(0)
    assert [f32_bits(float(v)) for v in vals] == [0x3EE214CA, 0xBE0F73A8, 0xBCAF4CC0, 0x3D350140]


def test_normal_constants_match_the_oracle_generator(mc, oracle):
    c = compile_none(mc, "const v : f32[1001] = normal(seed=7, mean=0.5, std=0.1)\noutput v\n", passes="none")
    assert np.array_equal(c.constant(0), oracle.normal(1001, 7, 0.5, 0.1))


# The reference's parser known answers, message for message
# (tests/test_parser.cpp:66-123).
REFERENCE_PARSE_ERRORS = [
    ("input x : f32[4]\ny = frobnicate x\noutput y", "line 2: unknown op 'frobnicate'"),
    ("input x : f32[4]\ny = relu z\noutput y", "line 2: unknown value 'z'"),
    ("input x : f32[4]\nx = relu x\noutput x", "line 2: 'x' is defined twice"),
    ("input x : i32[4]\noutput x", "line 1: unsupported element type 'i32' (only f32)"),
    ("input x : f32[N]\noutput x", "line 1: unknown dim 'N'"),
    ("const c : f32[3] = [1, 2]\noutput c", "line 1: expected 3 values for f32[3], got 2"),
    ("input x : f32[4]\n", "the graph declares no outputs"),
    ("input x : f32[4] ;", "line 1: unexpected character ';'"),
    ("input x : f32[4]\ny = relu x x", "line 2: unexpected 'x'"),
    ("const c : f32[-1] = 0\noutput c",
     "line 1: invalid shape [-1]: dimensions must be >= 1 and the total at most 2^31 - 1 elements"),
]
REFERENCE_INVALID_SHAPES = ["const c : f32[-1] = uniform(seed=1, lo=0, hi=1)\noutput c",
                            "input x : f32[7, 7905747460161236407]\noutput x",
                            "const c : f32[4294967296, 4294967296] = 1\noutput c",
                            "input x : f32[4, 0]\noutput x"]
REFERENCE_EXAMPLE = """
# A small MLP layer.
graph layer
dim B = 2
input x : f32[B, 3]
const w : f32[3, 4] = uniform(seed=7, lo=-0.5, hi=0.5)
const b : f32[4] = [1, 2, 3, 4]
const half : f32[] = 0.5
h = matmul x, w
hb = add h, b      # bias broadcast over rows
y = mul hb, half
output y, h
"""


def parse_error(mc, text, dims=None):
    try:
        compile_none(mc, text, passes="none", dims=dims)
    except mc.MinicompilerError as e:
        return str(e)
    return "<parsed>"


@pytest.mark.parametrize("text,message", REFERENCE_PARSE_ERRORS)
def test_parser_reports_the_reference_messages(mc, text, message):
    assert parse_error(mc, text) == message


def test_parser_rejects_invalid_shapes_before_allocating(mc):
    for text in REFERENCE_INVALID_SHAPES:
        assert parse_error(mc, text).startswith("line 1: invalid shape"), text


def test_parser_carries_ir_shape_errors_with_the_value_name(mc):
    err = parse_error(mc, "input a : f32[4, 8]\ninput b : f32[4]\nc = add a, b\noutput c")
    assert err.startswith("line 3: c: add: cannot broadcast"), err


def test_parser_reads_every_statement_kind_of_the_reference_example(mc, oracle):
    c = compile_none(mc, REFERENCE_EXAMPLE, passes="none")
    g = c.graph()
    assert g["name"] == "layer" and len(g["nodes"]) == 7 and c.num_inputs == 1 and c.num_outputs == 2
    assert node_named(g, "x")["shape"] == [2, 3] and node_named(g, "y")["shape"] == [2, 4]
    assert c.constant(node_named(g, "b")["id"]).tolist() == [1, 2, 3, 4]
    assert c.constant(node_named(g, "half")["id"]).tolist() == [0.5]
    assert np.array_equal(c.constant(node_named(g, "w")["id"]), oracle.uniform(12, 7, -0.5, 0.5))
    wide = compile_none(mc, REFERENCE_EXAMPLE, passes="none", dims={"B": 64})
    assert node_named(wide.graph(), "y")["shape"] == [64, 4]
    assert "no dim 'Q'" in parse_error(mc, REFERENCE_EXAMPLE, dims={"B": 64, "Q": 1})
    p = c.print_graph()
    assert "graph layer\n" in p
    assert "%0 x = input : f32[2,3]" in p
    assert "%2 b = const [1, 2, 3, 4] : f32[4]" in p
    assert "%6 y = mul %5, %3 : f32[2,4]  (output)" in p


def test_parser_keeps_large_seeds_exact(mc, oracle):
    a = compile_none(mc, "const c : f32[8] = uniform(seed=9007199254740992, lo=0, hi=1)\noutput c", passes="none")
    b = compile_none(mc, "const c : f32[8] = uniform(seed=9007199254740993, lo=0, hi=1)\noutput c", passes="none")
    assert not np.array_equal(a.constant(0), b.constant(0))
    assert np.array_equal(b.constant(0), oracle.uniform(8, 9007199254740993, 0.0, 1.0))


def test_parser_ignores_comments_blank_lines_and_carriage_returns(mc):
    c = compile_none(mc, "# header\r\n\r\ninput x : f32[2]   # trailing\r\ny = exp x\r\noutput y\r\n", passes="none")
    assert len(c.graph()["nodes"]) == 2


def test_parser_accepts_scalars_and_signed_numbers(mc):
    c = compile_none(mc, "const c : f32[] = -1.5e-1\nconst d : f32[2] = [-2, +.5]\ny = mul c, d\noutput y",
                     passes="none")
    g = c.graph()
    assert c.constant(node_named(g, "c")["id"]).tolist() == [np.float32(-0.15)]
    assert c.constant(node_named(g, "d")["id"]).tolist() == [-2.0, 0.5]


@pytest.mark.parametrize("text,needle", [
    ("const c : f32[2] = uniform(seed=1, lo=0)\noutput c", "missing 'hi'"),
    ("const c : f32[2] = uniform(seed=1, lo=0, lo=1, hi=2)\noutput c", "'lo' twice"),
    ("const c : f32[2] = uniform(seed=1, lo=0, mid=1, hi=2)\noutput c", "no argument 'mid'"),
    ("const c : f32[2] = uniform(seed=-1, lo=0, hi=2)\noutput c", "seed '-1'"),
    ("const c : f32[2] = normal(seed=1, mean=0, std=0)\noutput c", "std must be positive"),
    ("const c : f32[2] = poisson(seed=1)\noutput c", "no initializer named 'poisson'"),
    ("const c : f32[2] = 1e999\noutput c", "number '1e999'"),
    ("dim B = 1.5\ninput x : f32[B]\noutput x", "'1.5' is not a 64-bit integer"),
    ("dim B = 0\ninput x : f32[B]\noutput x", "not a positive size"),
    ("input x : f32[2]\ngraph late\noutput x", "has to precede every node"),
    ("input x : f32[2]\nfoo x\noutput x", "neither a statement keyword nor an assignment"),
    ("input x : f32[2\noutput x", "expected ',' or ']' before the end of the line"),
    ("input x f32[2]\noutput x", "expected ':' where 'f32' stands"),
])
def test_parser_names_what_is_wrong(mc, text, needle):
    assert needle in parse_error(mc, text), parse_error(mc, text)


def test_parser_terminates_on_random_text(mc):
    """Every text over the language's alphabet parses or fails (a lexer that
    stops advancing on some number form would hang here)."""
    rng = np.random.default_rng(5)
    pieces = ["input", "const", "dim", "output", "graph", "x", "y", "f32", ":", "=", ",", "[", "]", "(", ")",
              "0.5", ".5", "1.", "5.5.5", "1e", "1e-", "2E+3", "+", "-", "+.", "-.e", "..", "#c", "\n", " ", "\r",
              ";", "uniform", "seed=1", "relu", "add"]
    for _ in range(3000):
        text = "".join(rng.choice(pieces, size=int(rng.integers(1, 14))))
        parse_error(mc, text)
