"""Seeded random graphs as .mcg text, for fuzzing the passes and the backend.

Same idea as the reference's make_random_graph (tests/test_util.cpp:177-341):
grow a graph of unary, binary (every broadcasting pattern) and matmul nodes
over inputs and constants while tracking an interval bound for every value,
emitting an op only when it is numerically safe (log/sqrt of positive
values, divisors away from zero, no overflow). Dead values are left in place
(work for dead-node elimination) and some ops combine two constants (work
for constant folding). The random sequence is numpy's PCG64, not the
reference's mt19937_64, so the graphs differ; they are a fuzzer.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np


@dataclass
class Value:
    name: str
    shape: tuple
    lo: float
    hi: float
    const: bool

    @property
    def mag(self) -> float:
        return max(abs(self.lo), abs(self.hi))


def _bshape(a: tuple, b: tuple):
    rank = max(len(a), len(b))
    out = []
    for i in range(rank):
        da = a[len(a) - 1 - i] if i < len(a) else 1
        db = b[len(b) - 1 - i] if i < len(b) else 1
        if da != db and da != 1 and db != 1:
            return None
        out.append(db if da == 1 else da)
    return tuple(reversed(out))


def _fmt(x: float) -> str:
    return repr(float(x))


def make_random_graph(seed: int, num_ops: int = 16, allow_matmul: bool = True) -> str:
    rng = np.random.default_rng(seed)
    lines = [f"graph random_{seed}"]
    values: list[Value] = []
    counter = [0]
    const_seed = [seed * 7919]

    def pick(choices):
        return choices[int(rng.integers(len(choices)))]

    def fresh(prefix: str) -> str:
        counter[0] += 1
        return f"{prefix}{counter[0]}"

    def shape_text(s: tuple) -> str:
        return "f32[" + ", ".join(str(d) for d in s) + "]"

    def add_constant(name, shape, lo, hi):
        const_seed[0] += 1
        lines.append(f"const {name} : {shape_text(shape)} = uniform(seed={const_seed[0]}, lo={_fmt(lo)}, hi={_fmt(hi)})")
        values.append(Value(name, shape, float(np.float32(lo)), float(np.float32(hi)), True))

    m = pick([1, 2, 3, 7, 16, 33])
    n = pick([1, 4, 5, 8, 17, 64])
    lines.append(f"input x : {shape_text((m, n))}")
    values.append(Value("x", (m, n), -1, 1, False))
    if rng.random() < 0.7:
        lines.append(f"input y : {shape_text((m, n))}")
        values.append(Value("y", (m, n), -1, 1, False))
    if rng.random() < 0.5:
        lines.append(f"input row : {shape_text((n,))}")
        values.append(Value("row", (n,), -1, 1, False))
    if rng.random() < 0.5:
        lines.append(f"input col : {shape_text((m, 1))}")
        values.append(Value("col", (m, 1), -1, 1, False))
    add_constant("s", (), 0.5, 2.0)
    add_constant("bias", (n,), -1.0, 1.0)
    if rng.random() < 0.5:
        add_constant("pos", (m, n), 0.5, 1.5)
    leaves = len(values)

    def finish(op, args, shape, lo, hi, const):
        if not (max(abs(lo), abs(hi)) <= 1e3) or math.isnan(lo) or math.isnan(hi):
            return None
        name = fresh("v")
        lines.append(f"{name} = {op} {', '.join(a.name for a in args)}")
        return Value(name, shape, lo, hi, const)

    def try_unary():
        a = pick(values)
        op = pick(["neg", "exp", "log", "sqrt", "relu", "sigmoid", "tanh"])
        lo, hi = a.lo, a.hi
        if op == "neg":
            r = (-hi, -lo)
        elif op == "exp":
            if hi > 8.0:
                return None
            r = (math.exp(lo), math.exp(hi))
        elif op == "log":
            if lo < 0.05:
                return None
            r = (math.log(lo), math.log(hi))
        elif op == "sqrt":
            if lo < 0.0:
                return None
            r = (math.sqrt(lo), math.sqrt(hi))
        elif op == "relu":
            r = (max(lo, 0.0), max(hi, 0.0))
        elif op == "sigmoid":
            r = (1 / (1 + math.exp(-lo)), 1 / (1 + math.exp(-hi)))
        else:
            r = (math.tanh(lo), math.tanh(hi))
        return finish(op, [a], a.shape, r[0], r[1], a.const)

    def product(x, y):
        c = [x[0] * y[0], x[0] * y[1], x[1] * y[0], x[1] * y[1]]
        return min(c), max(c)

    def try_binary():
        a, b = pick(values), pick(values)
        if rng.random() < 0.15:
            consts = [v for v in values if v.const]
            a, b = pick(consts), pick(consts)
        shape = _bshape(a.shape, b.shape)
        if shape is None:
            return None
        op = pick(["add", "sub", "mul", "div"])
        x, y = (a.lo, a.hi), (b.lo, b.hi)
        if op == "add":
            r = (x[0] + y[0], x[1] + y[1])
        elif op == "sub":
            r = (x[0] - y[1], x[1] - y[0])
        elif op == "mul":
            r = product(x, y)
        else:
            if y[0] < 0.1 and y[1] > -0.1:
                return None
            r = product(x, (1.0 / y[1], 1.0 / y[0]))
        return finish(op, [a, b], shape, r[0], r[1], a.const and b.const)

    def try_matmul():
        a = pick(values)
        if len(a.shape) != 2:
            return None
        k = a.shape[1]
        cols = pick([1, 3, 8, k])
        w = 1.0 / math.sqrt(k)
        name = fresh("w")
        add_constant(name, (k, cols), -w, w)
        weight = values.pop()
        bound = k * a.mag * w
        v = finish("matmul", [a, weight], (a.shape[0], cols), -bound, bound, a.const)
        values.append(weight)
        return v

    created = 0
    attempts = 0
    while created < num_ops and attempts < num_ops * 50:
        attempts += 1
        r = rng.random()
        if r < 0.40:
            v = try_unary()
        elif r < 0.88 or not allow_matmul:
            v = try_binary()
        else:
            v = try_matmul()
        if v is not None:
            values.append(v)
            created += 1

    computed = [v for v in values[leaves:] if not v.name.startswith("w")]
    outputs = []
    if computed:
        outputs.append(computed[-1].name)
    else:
        lines.append("negx = neg x")
        outputs.append("negx")
    for _ in range(int(rng.integers(3))):
        if computed:
            cand = pick(computed).name
            if cand not in outputs:
                outputs.append(cand)
    lines.append("output " + ", ".join(outputs))
    return "\n".join(lines) + "\n"
