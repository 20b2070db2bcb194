"""mc_launch_matmul_noalloc (the GEMM operator with its split-K partials in
the library's per-GPU scratch array, for callers that cannot allocate)
against mc_launch_matmul with a caller workspace, through the C ABI: the
same kernels, so the same bits. Each case makes two calls in a row on the
shared array, the second on a smaller product, and a product whose partials
exceed the array is refused with a message. The first call of a process
(the one that looks up the array's device address) can be captured into a
HIP graph: checked in a child process, so that it is that process's first.
"""

import os
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

# (kernel, [(m, k, n, splits) first call, second smaller call])
CASES = [
    ("split_k", [(512, 8192, 512, 16), (128, 2048, 256, 8)]),
    ("split_k", [(256, 16384, 256, 64), (16, 4096, 4096, 8)]),
    ("tensor_core_bf16", [(300, 4096, 264, 4), (64, 512, 64, 2)]),
    ("tensor_core_f16", [(256, 2048, 512, 8), (33, 256, 40, 3)]),
    ("double_buffered", [(1024, 1024, 1024, 1), (96, 256, 100, 1)]),
]


def run_pair(mc, oracle, kernel, m, k, n, splits, seed):
    a = oracle.uniform(m * k, seed, -1.0, 1.0)
    b = oracle.uniform(k * n, seed + 1, -1.0, 1.0)
    da, db = mc.DeviceBuffer.from_array(a), mc.DeviceBuffer.from_array(b)
    nan = np.full(m * n, np.nan, dtype=np.float32)
    c_ws, c_na = mc.DeviceBuffer.from_array(nan), mc.DeviceBuffer.from_array(nan)
    ws_bytes = mc.matmul_workspace_bytes(kernel, m, n, splits)
    ws = mc.DeviceBuffer(ws_bytes) if ws_bytes > 0 else None
    mc.launch_matmul(kernel, da.ptr, db.ptr, c_ws.ptr, m, n, k, None, splits, ws.ptr if ws else None)
    mc.launch_matmul_noalloc(kernel, da.ptr, db.ptr, c_na.ptr, m, n, k, None, splits)
    mc.synchronize()
    want, got = c_ws.download(), c_na.download()
    assert not np.any(np.isnan(got)), "an element of C was not written"
    return want, got


@pytest.mark.parametrize("kernel,calls", CASES)
def test_noalloc_matmul_equals_the_workspace_entry_point_on_two_calls(device, mc, oracle, kernel, calls):
    for i, (m, k, n, splits) in enumerate(calls):
        print(f"case noalloc {kernel} {m}x{k}x{n} splits={splits} call {i}", flush=True)
        want, got = run_pair(mc, oracle, kernel, m, k, n, splits, 3 + 2 * i)
        assert np.array_equal(want.view(np.uint32), got.view(np.uint32)), f"call {i}: bits differ"


def test_noalloc_matmul_refuses_partials_beyond_its_scratch(device, mc, oracle):
    cap = mc.noalloc_scratch_bytes()
    assert cap == 32 << 20
    m = n = 512
    splits = 64  # 64 MiB of partials
    assert mc.matmul_workspace_bytes("split_k", m, n, splits) > cap
    print("case noalloc refusal 512x4096x512 splits=64", flush=True)
    da = mc.DeviceBuffer(4 * m * 4096)
    db = mc.DeviceBuffer(4 * 4096 * n)
    dc = mc.DeviceBuffer.from_array(np.full(m * n, np.nan, dtype=np.float32))
    with pytest.raises(mc.HipError, match="more than the library's 33554432-byte scratch"):
        mc.launch_matmul_noalloc("split_k", da.ptr, db.ptr, dc.ptr, m, n, 4096, None, splits)
    mc.synchronize()
    assert np.all(np.isnan(dc.download())), "a refused call must not launch"


REPO = Path(__file__).resolve().parents[1]
SCRIPT = r"""
import sys
import numpy as np
sys.path.insert(0, {repo!r})
import minicompiler_amd as mc
m, k, n, splits = 256, 4096, 256, 8
a, b = mc.uniform(m * k, 5, -1.0, 1.0), mc.uniform(k * n, 6, -1.0, 1.0)
da, db = mc.DeviceBuffer.from_array(a), mc.DeviceBuffer.from_array(b)
nan = np.full(m * n, np.nan, dtype=np.float32)
c_na, c_ws = mc.DeviceBuffer.from_array(nan), mc.DeviceBuffer.from_array(nan)
ws = mc.DeviceBuffer(mc.matmul_workspace_bytes("split_k", m, n, splits))
s = mc.Stream()
print("capturing the first no-allocation call", flush=True)
g = mc.CapturedGraph(s, lambda st: mc.launch_matmul_noalloc("split_k", da.ptr, db.ptr, c_na.ptr, m, n, k, st, splits))
mc.launch_matmul("split_k", da.ptr, db.ptr, c_ws.ptr, m, n, k, None, splits, ws.ptr)
mc.synchronize()
want = c_ws.download().view(np.uint32)
for rep in range(3):
    c_na.upload(nan)
    g.launch()
    s.synchronize()
    got = c_na.download()
    assert not np.any(np.isnan(got)), f"replay {{rep}}: an element of C was not written"
    assert np.array_equal(got.view(np.uint32), want), f"replay {{rep}}: bits differ"
    mc.launch_matmul("split_k", da.ptr, db.ptr, c_ws.ptr, m, n, k, None, splits, ws.ptr)
    mc.synchronize()
print("capture ok", flush=True)
"""


def test_the_first_noalloc_call_can_be_captured_into_a_graph(device):
    print("case noalloc first call under capture (child process)", flush=True)
    r = subprocess.run([sys.executable, "-c", SCRIPT.format(repo=str(REPO))], env=dict(os.environ),
                       capture_output=True, text=True, timeout=150)
    assert r.returncode == 0, r.stdout[-1000:] + r.stderr[-2000:]
    assert "capture ok" in r.stdout
