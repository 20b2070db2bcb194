"""The oracle and this build's host logic against the reference's own known
answers (tests/golden/reference_known_answers.json, transcribed from the
reference's tests with file:line). CPU only."""

import json
import struct
from pathlib import Path

import numpy as np
import pytest

GOLDEN = json.loads((Path(__file__).parent / "golden" / "reference_known_answers.json").read_text())


def bits(x: float) -> int:
    return struct.unpack("<I", struct.pack("<f", x))[0]


def test_rng_golden_bits_in_the_oracle_and_the_library(oracle, mc):
    for case in GOLDEN["rng_uniform"]:
        want = [int(b, 16) for b in case["bits"]]
        got = oracle.uniform(case["count"], case["seed"], case["lo"], case["hi"])
        assert [bits(float(v)) for v in got] == want, case["source"]
        assert [bits(float(v)) for v in mc.uniform(case["count"], case["seed"], case["lo"], case["hi"])] == want


@pytest.mark.parametrize("case", GOLDEN["stage_counts"], ids=lambda c: c["graph"])
def test_stage_counts(mc, case):
    c = mc.Compiled(path=mc.graph_path(case["graph"]), dims=case["dims"], backend="none")
    counts = [[s["stats"]["nodes"], s["stats"]["compute_nodes"]] for s in c.stage_stats()]
    assert counts == case["counts"], case["source"]
    last = c.stage_stats()[-1]["stats"]
    for key in ("fused_nodes", "elementwise_ops", "matmuls"):
        if key in case:
            assert last[key] == case[key], (key, case["source"])


def test_constant_folding_known_answers(mc):
    g = GOLDEN["constant_folding"]
    c = g["sqrt_2_over_pi"]
    text = (f"input x : f32[4]\nconst two : f32[] = {c['two']}\nconst pi : f32[] = {c['pi']}\n"
            "ratio = div two, pi\nc = sqrt ratio\ny = mul x, c\noutput y\n")
    comp = mc.Compiled(text, passes="fold", backend="none")
    graph = comp.graph()
    node = next(n for n in graph["nodes"] if n["name"] == "c")
    assert node["op_name"] == "const"
    assert abs(float(comp.constant(node["id"])[0]) - np.sqrt(2.0 / c["pi"])) <= c["tolerance"]
    bn = g["batchnorm"]
    fmt = lambda v: ", ".join(repr(float(x)) for x in v)
    text = (f"input x : f32[2, 3]\nconst var : f32[3] = [{fmt(bn['var'])}]\nconst eps : f32[] = {bn['eps']}\n"
            f"const gamma : f32[3] = [{fmt(bn['gamma'])}]\nconst w : f32[2, 3] = [{fmt(bn['w'])}]\n"
            f"const m : f32[2, 2] = [{fmt(bn['m'])}]\n"
            "ve = add var, eps\nsd = sqrt ve\nscale = div gamma, sd\nws = mul w, scale\nsq = matmul m, ws\n"
            "y = add x, sq\noutput y\n")
    comp = mc.Compiled(text, passes="fold", backend="none")
    nodes = {n["name"]: n for n in comp.graph()["nodes"]}
    for name in ("scale", "ws", "sq"):
        assert nodes[name]["op_name"] == "const", name
        assert comp.constant(nodes[name]["id"]).tolist() == bn[name], (name, g["source"])
    assert nodes["y"]["op_name"] == "add"


def test_chain_buffer_counts(mc):
    for case in GOLDEN["chain_buffers"]:
        n, length = case["elements"], case["length"]
        text = f"input x : f32[{n}]\n" + "".join(
            f"v{i + 1} = tanh {'x' if i == 0 else f'v{i}'}\n" for i in range(length)) + f"output v{length}\n"
        c = mc.Compiled(text, passes="none", backend="none")
        plan = c.plan(pool_outputs=True)
        if "buffers" in case:
            assert len(plan["buffer_bytes"]) == case["buffers"], case["source"]
            assert plan["bytes_without_reuse"] == case["bytes_without_reuse"]
            assert sum(plan["buffer_bytes"]) == case["bytes_with_reuse"]
        else:
            assert c.intermediate_bytes == case["intermediate_bytes"], case["source"]


def test_split_rule_workspace_and_resolution(mc):
    for m, n, k, sms, bps, want in GOLDEN["split_k_splits"]["cases"]:
        assert mc.split_k_splits(m, n, k, sms, bps) == want, (m, n, k, sms, bps)
    for kernel, m, n, splits, want in GOLDEN["workspace_bytes"]["cases"]:
        assert mc.matmul_workspace_bytes(kernel, m, n, splits) == want, (kernel, m, n, splits)
    for kernel, m, n, k, sms, want in GOLDEN["resolve_auto"]["cases"]:
        assert mc.resolve_matmul_kernel(kernel, m, n, k, sms) == want, (kernel, m, n, k, sms)


def test_generator_known_answers(mc):
    g = GOLDEN["codegen"]
    for value, want in g["immediate_bits"]:
        v = float("inf") if value == "inf" else value
        src, _ = mc.generate_elementwise_kernel(f"r0 = load in0\nr1 = imm {v}\nr2 = mul r0, r1\n", [(8,)], (8,))
        assert f"__uint_as_float({want}u)" in src, (value, want)
    for case in g["periodic"] + g["general"]:
        src, vec = mc.generate_elementwise_kernel("r0 = load in0\nr1 = load in1\nr2 = mul r0, r1\n",
                                                  case["shapes"], case["out"])
        assert case["index"] in src, case
        if "vectorized" in case:
            assert vec == case["vectorized"]
    for count, want in g["vectorized_by_count"]:
        _, vec = mc.generate_elementwise_kernel("r0 = load in0\nr1 = load in1\nr2 = div r0, r1\n", [(count,), ()],
                                                (count,))
        assert vec == want, count
