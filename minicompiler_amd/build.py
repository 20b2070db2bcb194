"""Builds libminicompiler_hip.so (and the mcc driver) in-tree.

Host C++ (the compiler core, the HIP backend's host side and the C ABI) is
compiled with g++ and sees no HIP header except in the thin layer
csrc/hip/hip_rt.cpp. The matmul kernels (csrc/hip/*.hip) are compiled
ahead of time for gfx950 with hipcc. Everything links into one shared
library against libamdhip64 and libhiprtc. Always rebuilds everything (the
"does it build" check must compile), in parallel.

    python -m minicompiler_amd.build            # library + mcc
"""

from __future__ import annotations

import concurrent.futures as futures
import os
import shlex
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
BUILD = ROOT / "_build" / "minicompiler_amd"
LIBDIR = PKG / "lib"
LIBRARY = LIBDIR / "libminicompiler_hip.so"
MCC = PKG / "bin" / "mcc"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
ARCH = "gfx950"

CXXFLAGS = ["-std=c++17", "-O2", "-fPIC", "-Wall", "-Wextra", "-Wno-unused-parameter", "-ffp-contract=off",
            f"-I{INCLUDE}", f"-I{CSRC}"]
# Kernels: gfx950 only; packed FP32 instructions off (see the build notes).
HIPFLAGS = ["-std=c++17", "-O3", "-fPIC", f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang",
            "-packed-fp32-ops", "-Wno-unused-command-line-argument", f"-I{INCLUDE}", f"-I{CSRC}"]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature.
    lines = [l for l in proc.stdout.splitlines() if "packed-fp32-ops' is not a recognized feature" not in l]
    if proc.returncode != 0:
        raise RuntimeError("build step failed:\n" + " ".join(shlex.quote(c) for c in cmd) + "\n" + "\n".join(lines))
    if lines:
        print("\n".join(lines), file=sys.stderr)


def _sources() -> tuple[list[Path], list[Path], Path]:
    host = sorted((CSRC / "core").glob("*.cpp")) + sorted((CSRC / "hip").glob("*.cpp")) + [CSRC / "capi.cpp"]
    kernels = sorted((CSRC / "hip").glob("*.hip"))
    return host, kernels, CSRC / "tools" / "mcc.cpp"


def _object(src: Path) -> Path:
    rel = src.relative_to(CSRC)
    return BUILD / (str(rel).replace("/", "__") + ".o")


def _compile(src: Path) -> Path:
    obj = _object(src)
    obj.parent.mkdir(parents=True, exist_ok=True)
    if src.suffix == ".hip":
        cmd = [str(ROCM / "bin" / "hipcc"), *HIPFLAGS, "-c", str(src), "-o", str(obj)]
    else:
        cmd = ["g++", *CXXFLAGS]
        if src.name == "hip_rt.cpp":  # the one host file that includes HIP headers
            cmd += [f"-I{ROCM / 'include'}", "-D__HIP_PLATFORM_AMD__"]
        cmd += ["-c", str(src), "-o", str(obj)]
    _run(cmd)
    return obj


def build(jobs: int | None = None, verbose: bool = True) -> Path:
    host, kernels, mcc = _sources()
    jobs = jobs or min(16, os.cpu_count() or 4)
    # Kernel TUs first in the queue: they take the longest.
    order = kernels + host
    with futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(_compile, order))
    LIBDIR.mkdir(parents=True, exist_ok=True)
    tmp = LIBRARY.with_suffix(".so.tmp")
    _run([str(ROCM / "bin" / "hipcc"), "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", str(tmp), *map(str, objs),
          f"-L{ROCM / 'lib'}", "-lamdhip64", "-lhiprtc", f"-Wl,-rpath,{ROCM / 'lib'}", "-Wl,--no-undefined"])
    os.replace(tmp, LIBRARY)
    MCC.parent.mkdir(parents=True, exist_ok=True)
    _run(["g++", *CXXFLAGS, str(mcc), "-o", str(MCC), f"-L{LIBDIR}", "-lminicompiler_hip",
          "-Wl,-rpath,$ORIGIN/../lib", f"-Wl,-rpath,{ROCM / 'lib'}"])
    if verbose:
        print(f"built {LIBRARY.relative_to(ROOT)} and {MCC.relative_to(ROOT)}")
    return LIBRARY


if __name__ == "__main__":
    build()
