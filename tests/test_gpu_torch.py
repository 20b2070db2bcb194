"""Compiled graphs bound to PyTorch tensors and enqueued on PyTorch's stream,
as the reference's harness runs them beside PyTorch (bench/capi.cpp:150-158,
bench/torch_compare.py:188-214): inputs and outputs are PyTorch CUDA
tensors (mc_bind_inputs / mc_bind_outputs), the launches go on PyTorch's
current stream (mc_enqueue), and PyTorch work queued before and after them
on that stream is ordered with them. The outputs must match the CPU oracle
(rtol 1e-5 plus 1e-5 of the scale for elementwise graphs, 1e-4 with FP32
GEMMs) and PyTorch's own library ops on the same tensors (normwise 1e-4,
torch_compare's agreement bar).

The check runs in one child process (tests/torch_stream_check.py) that
imports PyTorch before the library: PyTorch ships its own HIP runtime under
the same soname, and in this process the library's was loaded first."""

import json
import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu


def test_graphs_on_pytorch_tensors_and_stream_match_the_oracle_and_pytorch(device):
    pytest.importorskip("torch")
    script = Path(__file__).resolve().parent / "torch_stream_check.py"
    proc = subprocess.run([sys.executable, "-u", str(script)], capture_output=True, text=True, timeout=240)
    sys.stderr.write(proc.stderr[-4000:])
    results = [json.loads(line) for line in proc.stdout.splitlines() if line.startswith("{")]
    for r in results:
        print(r if r.get("ok") else r.get("error"), flush=True)
    assert proc.returncode == 0, [r for r in results if not r.get("ok")] or proc.stderr[-2000:]
    assert len(results) == 4 and all(r["ok"] for r in results)
