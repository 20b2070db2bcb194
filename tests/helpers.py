"""Shared test helpers: tolerance checks (the reference's all_close,
tests/test_util.cpp:12-43), seeded inputs, and the GEMM error bounds."""

from __future__ import annotations

import math

import numpy as np

U32 = 2.0 ** -24


def all_close(actual, expected, rtol: float, atol: float) -> tuple[bool, str]:
    """|actual - expected| <= atol + rtol |expected| elementwise; NaN matches
    NaN and equal infinities match. On failure names the worst element."""
    a = np.asarray(actual, dtype=np.float64).reshape(-1)
    e = np.asarray(expected, dtype=np.float64).reshape(-1)
    if a.shape != e.shape:
        return False, f"size {a.size} vs expected {e.size}"
    with np.errstate(invalid="ignore"):
        equal = (a == e) | (np.isnan(a) & np.isnan(e))
        err = np.abs(a - e)
        allowed = atol + rtol * np.abs(e)
        bad = ~equal & ~(err <= allowed)
    if not bad.any():
        return True, ""
    with np.errstate(divide="ignore", invalid="ignore"):
        ratio = np.where(bad, np.where(allowed > 0, err / allowed, np.inf), -1.0)
    w = int(np.nanargmax(np.where(np.isnan(ratio), np.inf, ratio)))
    return False, (f"{int(bad.sum())} of {a.size} elements differ; worst at [{w}]: actual {a[w]!r}, "
                   f"expected {e[w]!r} (rtol {rtol}, atol {atol})")


def assert_close(actual, expected, rtol: float, atol: float, what: str = "") -> None:
    ok, msg = all_close(actual, expected, rtol, atol)
    assert ok, f"{what}: {msg}" if what else msg


def max_abs(x) -> float:
    x = np.asarray(x, dtype=np.float64)
    return float(np.max(np.abs(x))) if x.size else 0.0


def gamma(k: int) -> float:
    return k * U32 / (1.0 - k * U32)


def fp32_gemm_bound(exact_or_cpu, absdot, k: int) -> np.ndarray:
    """Two fp32 dot products of length k each lie within gamma_k sum|ab| of
    the exact one, so they differ by at most twice that plus each side's
    final rounding (tests/test_cuda_backend.cpp:119-159)."""
    return 2.0 * gamma(k) * absdot + 2.0 * U32 * np.abs(exact_or_cpu)


def lowp_gemm_bound(exact, absdot, k: int, u: float, subnormals: bool) -> np.ndarray:
    """Inputs rounded to a format of unit roundoff u: each product within
    (2u + u^2)|ab|; FP32 accumulation adds gamma_k sum|ab|, doubled; plus the
    final rounding; fp16 loses up to 2^-25 per rounded input below its
    smallest normal (tests/test_cuda_backend.cpp:164-219)."""
    tiny = 2.0 * k * 2.0 ** -25 if subnormals else 0.0
    return (2.0 * u + u * u + 2.0 * gamma(k)) * absdot + 2.0 * U32 * np.abs(exact) + tiny


def uniform_inputs(oracle, sizes, seed: int, lo: float = -1.0, hi: float = 1.0) -> list[np.ndarray]:
    """Input k = uniform(n_k, seed + k, lo, hi), as make_random_inputs does
    (src/runtime/host_tensor.cpp:7-14)."""
    return [oracle.uniform(int(n), seed + k, lo, hi) for k, n in enumerate(sizes)]


def run_into_prefilled(mc, compiled, inputs) -> list[np.ndarray]:
    """Runs `compiled` on `inputs` with every output bound to a device
    buffer whose bytes are all 0xFF (a NaN in every float), so an element the
    kernels never write reads back as NaN (the reference's NaN prefill,
    tests/test_cuda_backend.cpp:297). Returns the outputs as float32 arrays."""
    bufs = [mc.DeviceBuffer(4 * n) for n in compiled.output_sizes]
    for b in bufs:
        b.fill_bytes(0xFF)
    compiled.bind_outputs([b.ptr for b in bufs])
    compiled.upload(inputs)
    compiled.enqueue()
    compiled.synchronize()
    outs = [b.download() for b in bufs]
    compiled.bind_outputs([None] * len(bufs))
    return outs


def row_blocks(total: int, rows: int, seed: int, middle: int = 2) -> list[int]:
    """First rows of the blocks a full-size check compares: the first and the
    last `rows` rows, plus `middle` seeded starts in between (not aligned to
    a tile, so each straddles a tile boundary)."""
    rng = np.random.default_rng(seed)
    mids = sorted(int(s) for s in rng.integers(rows, total - 2 * rows, middle))
    return [0] + mids + [total - rows]
