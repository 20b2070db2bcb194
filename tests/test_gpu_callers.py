"""The reference's other callers of the backend, on the GPU:

- the driver: `mcc GRAPH --dim ... --backend hip --run` (tools/mcc.cpp:
  213-238) prints each output's sum and sum of magnitudes over seeded
  uniform(-1, 1) inputs (input k from seed 1 + k, host_tensor.cpp:7-14) and
  writes the outputs with --dump-outputs; both are checked against the CPU
  oracle on the same inputs;
- the C-ABI harness enqueueing on a stream the caller made
  (bench/capi.cpp:150-158): mc_upload, mc_enqueue on a stream from
  mc_stream_create (not the executable's own), then mc_download, against
  the oracle; twice, with other inputs the second time."""

import subprocess

import numpy as np
import pytest

from helpers import assert_close, max_abs, uniform_inputs

pytestmark = pytest.mark.gpu

MCC_CASES = [("gelu_chain", {"M": 4096, "N": 4096}, [], 1e-5), ("mlp_gelu", {"B": 256}, [], 1e-4),
             ("batchnorm_relu", {"R": 2048, "C": 256}, [], 1e-5),
             ("matmul_bias_relu", {}, ["--matmul", "split_k"], 1e-4)]


@pytest.mark.parametrize("name,dims,extra,rtol", MCC_CASES)
def test_mcc_run_matches_the_oracle(device, mc, oracle, tmp_path, name, dims, extra, rtol):
    exe = mc.PACKAGE_DIR / "bin" / "mcc"
    assert exe.exists(), "mcc is built by __graft_entry__.build()"
    dump = tmp_path / "out.bin"
    cmd = [str(exe), str(mc.graph_path(name)), "--backend", "hip", "--run", "--dump-outputs", str(dump), *extra]
    for k, v in dims.items():
        cmd += ["--dim", f"{k}={v}"]
    print("case mcc " + " ".join(cmd[1:]), flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    lines = [ln for ln in r.stdout.splitlines() if ln.startswith("output ")]
    part = mc.Compiled(path=mc.graph_path(name), dims=dims, backend="none")
    assert len(lines) == part.num_outputs
    inputs = uniform_inputs(oracle, part.input_sizes, 1)
    cpu = oracle.evaluate_compiled(part, inputs)
    data = np.fromfile(dump, dtype=np.float32)
    assert data.size == sum(part.output_sizes)
    at = 0
    for line, c in zip(lines, cpu):
        got = data[at:at + c.size]
        at += c.size
        assert_close(got, c, rtol, rtol * max(1.0, max_abs(c)), f"mcc {name}")
        # The printed checksums are the dumped outputs'.
        fields = line.replace(",", "").split()
        s, sa = float(fields[fields.index("sum") + 1]), float(fields[fields.index("sum|x|") + 1])
        g64 = got.astype(np.float64)
        assert s == pytest.approx(float(np.sum(g64)), rel=1e-6, abs=1e-6)
        assert sa == pytest.approx(float(np.sum(np.abs(g64))), rel=1e-6)
        # And within the tolerance's reach of the oracle's.
        assert sa == pytest.approx(float(np.sum(np.abs(c.astype(np.float64)))), rel=10 * rtol)


STREAM_CASES = [("mlp_gelu", {"B": 1024}, {}, 1e-4), ("gelu_chain", {"M": 512, "N": 4096}, {}, 1e-5),
                ("mlp_gelu", {"B": 256}, {"matmul": "split_k"}, 1e-4)]


@pytest.mark.parametrize("name,dims,opts,rtol", STREAM_CASES)
def test_enqueue_on_a_caller_stream_then_download(device, mc, oracle, name, dims, opts, rtol):
    print(f"case caller stream {name} {dims} {opts}", flush=True)
    c = mc.Compiled(path=mc.graph_path(name), dims=dims, options=opts)
    stream = mc.Stream()
    assert stream.handle and stream.handle != c.stream
    for rep in range(2):
        inputs = uniform_inputs(oracle, c.input_sizes, 30 + rep)
        c.upload(inputs)
        c.enqueue(stream)
        got = c.download()  # waits for the device, then copies
        cpu = oracle.evaluate_compiled(c, inputs)
        for g, w in zip(got, cpu):
            assert_close(g, w, rtol, rtol * max(1.0, max_abs(w)), f"caller stream, run {rep}")
    # Enqueued on the caller's stream, ordered behind that stream's earlier
    # work and waited for by that stream's synchronisation.
    out = mc.DeviceBuffer(4 * c.output_sizes[0])
    out.fill_bytes(0xFF)
    c.bind_outputs([out.ptr] + [None] * (c.num_outputs - 1))
    c.enqueue(stream)
    stream.synchronize()
    assert np.array_equal(out.download().view(np.uint32), got[0].view(np.uint32))
