"""Builds the CPU oracle (TEST INFRASTRUCTURE ONLY) into oracle/liboracle.so.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it.
x86-64-v3 (AVX2, FMA) so the library runs on any current x86 host. The
elementwise code is built without FP contraction (each op rounds to float);
the GEMM translation unit allows fused multiply-adds.

    python -m oracle.build
"""

from __future__ import annotations

import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"
BUILD = HERE.parent / "_build" / "oracle"
COMMON = ["g++", "-std=c++17", "-O3", "-fPIC", "-march=x86-64-v3", "-Wall", "-Wextra", f"-I{HERE}"]


def build(verbose: bool = True) -> Path:
    BUILD.mkdir(parents=True, exist_ok=True)
    objs = []
    for src, flags in (("cpu_oracle.cpp", ["-ffp-contract=off"]), ("cpu_gemm.cpp", ["-ffp-contract=fast"])):
        obj = BUILD / (src + ".o")
        subprocess.run([*COMMON, *flags, "-c", str(HERE / src), "-o", str(obj)], check=True)
        objs.append(str(obj))
    tmp = LIB.with_suffix(".so.tmp")
    subprocess.run(["g++", "-shared", "-o", str(tmp), *objs, "-lpthread"], check=True)
    tmp.replace(LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build()
