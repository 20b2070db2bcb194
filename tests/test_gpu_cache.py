"""The on-disk code-object cache (MINICOMPILER_HIP_CACHE_DIR): a second
process finds every generated kernel on disk (no hipRTC compile) and gets
the same results; a cache file whose stored key differs from the one asked
for is not used. (The reference's cache is in memory only,
src/cuda/kernel_compiler.cpp:24-57; the disk cache is this build's.)"""

import json
import os
import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

REPO = Path(__file__).resolve().parents[1]
SCRIPT = """
import json, sys
import numpy as np
sys.path.insert(0, {repo!r})
import minicompiler_amd as mc
c = mc.Compiled(path=mc.graph_path("mlp_gelu"), dims={{"B": 256}})
x = mc.uniform(c.input_sizes[0], 5, -1.0, 1.0)
y = c.run([x])[0]
print(json.dumps({{"jit_ms": c.jit_compile_ms, "sources": len(c.kernel_sources),
                  "sum": float(np.sum(y.astype(np.float64))), "bits": int(np.bitwise_xor.reduce(y.view(np.uint32)))}}))
"""


def run_child(cache_dir: Path) -> dict:
    env = {**os.environ, "MINICOMPILER_HIP_CACHE_DIR": str(cache_dir)}
    print(f"case cache child {cache_dir}", flush=True)
    r = subprocess.run([sys.executable, "-c", SCRIPT.format(repo=str(REPO))], env=env, capture_output=True, text=True,
                       timeout=150)
    assert r.returncode == 0, r.stderr[-2000:]
    return json.loads(r.stdout.strip().splitlines()[-1])


def test_second_process_loads_kernels_from_disk_and_rejects_a_foreign_key(device, tmp_path):
    first = run_child(tmp_path)
    files = sorted(tmp_path.glob("mc_*.co"))
    assert first["jit_ms"] > 0 and len(files) >= 1
    second = run_child(tmp_path)
    assert second["jit_ms"] == 0.0
    assert (second["sum"], second["bits"]) == (first["sum"], first["bits"])
    # Change one byte of the stored key in every file: none may be used.
    for f in files:
        data = bytearray(f.read_bytes())
        nl = data.index(b"\n")              # end of the magic line
        nl2 = data.index(b"\n", nl + 1)     # end of the key length
        data[nl2 + 1] ^= 0x01               # first byte of the key
        f.write_bytes(bytes(data))
    third = run_child(tmp_path)
    assert third["jit_ms"] > 0
    assert (third["sum"], third["bits"]) == (first["sum"], first["bits"])
    assert not list(tmp_path.glob("*.tmp*")), "a temporary file was left behind"


def test_a_truncated_code_object_is_a_miss_and_is_compiled_again(device, tmp_path):
    # Each file records its code object's length and hash: a torn or cut-off
    # write is recompiled (and the file rewritten), not loaded.
    first = run_child(tmp_path)
    files = sorted(tmp_path.glob("mc_*.co"))
    assert files
    for f in files:
        data = f.read_bytes()
        f.write_bytes(data[:-100])
    second = run_child(tmp_path)
    assert second["jit_ms"] > 0
    assert (second["sum"], second["bits"]) == (first["sum"], first["bits"])
    third = run_child(tmp_path)
    assert third["jit_ms"] == 0.0, "the rewritten files load again"
    assert not list(tmp_path.glob("*.tmp*"))
