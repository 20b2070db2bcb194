"""bench.py's stdout line (host logic, no GPU): the record a harness parses
may be only the last few thousand characters of stdout, so the one JSON
line bench.py prints stays below SUMMARY_MAX_BYTES and carries the headline
fields, `roofline` (with `traffic`) and `cpu_baseline`, while every config's
detail goes to the --out file. Checked on a full record a real bench run
wrote (tests/golden/bench_full_record.json) and on a synthetic worst case."""

import copy
import json
import sys
from pathlib import Path

import pytest

sys.path.insert(0, str(Path(__file__).resolve().parents[1]))

import bench  # noqa: E402

FIXTURE = Path(__file__).resolve().parent / "golden" / "bench_full_record.json"
HEADLINE = ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better", "scaling",
            "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline")


def recorded() -> dict:
    return json.loads(FIXTURE.read_text())


def check_line(full: dict) -> dict:
    line = bench.summary_line(full)
    text = json.dumps(line)
    assert len(text.encode()) < bench.SUMMARY_MAX_BYTES
    assert json.loads(text) == line
    for key in HEADLINE:
        assert key in line, key
    for key in ("bound", "achieved", "peak", "unit", "frac", "traffic"):
        assert key in line["roofline"], key
    for key in ("value", "unit", "cores", "kind", "sample"):
        assert key in line["cpu_baseline"], key
    assert line["value"] == full["value"] and line["roofline"] == full["roofline"]
    return line


def test_the_recorded_run_fits_with_every_config():
    full = recorded()
    assert len(json.dumps(full)) > bench.SUMMARY_MAX_BYTES, "the fixture is a full record"
    line = check_line(full)
    assert set(line["configs"]) == set(bench.summary_configs(full["configs"]))
    for name in ("gelu_4096x4096", "batchnorm_relu_200704x256", "gelu_fusion_4096x4096", "mlp_b256", "mlp_b1024",
                 "gemm_fp32", "gemm_bf16_fp16", "gemm_bf16_fp16_bias_gelu"):
        assert name in line["configs"], name
    assert len(line["configs"]["gemm_fp32"]["rows"]) == 6
    assert line["configs"]["gelu_4096x4096"]["cpu"]["value"] > 0


def test_an_oversized_record_drops_configs_before_the_headline():
    full = recorded()
    big = copy.deepcopy(full)
    # Forty times the GEMM rows, with long names: far past the limit.
    rows = big["configs"]["gemm_fp32"]
    big["configs"]["gemm_fp32"] = [dict(e, m=e["m"] + i) for i in range(40) for e in rows]
    line = check_line(big)
    assert "configs" not in line
    assert line["kernels"], "the headline's launches stay"


def test_long_cpu_samples_are_cut():
    full = recorded()
    full["cpu_baseline"]["sample"] = "x" * 5000
    line = check_line(full)
    assert len(line["cpu_baseline"]["sample"]) <= 240


@pytest.mark.parametrize("workload", ["gelu", "gemm_bf16"])
def test_single_workload_records_fit(workload):
    full = recorded()
    keep = {"gelu": ["gelu_4096x4096", "gelu_fusion_4096x4096"], "gemm_bf16": ["gemm_bf16_fp16"]}[workload]
    full["configs"] = {k: v for k, v in full["configs"].items() if k in keep}
    check_line(full)


def test_bf16_rows_keep_each_a_layout_apart():
    # The bf16/fp16 GEMM rows come in two A layouts (row-major, packed); the
    # summary keys them apart, and both still fit.
    full = recorded()
    rows = full["configs"]["gemm_bf16_fp16"]
    full["configs"]["gemm_bf16_fp16"] = [dict(e, a_layout=layout) for e in rows for layout in ("row-major", "packed")]
    line = check_line(full)
    keys = list(line["configs"]["gemm_bf16_fp16"]["rows"])
    assert len(keys) == 2 * len(rows)
    assert "bf16 8192x8192x8192" in keys and "bf16 8192x8192x8192 A packed" in keys


def test_the_counted_kernels_match_the_bench_lines_workload_names():
    # roofline.traffic is looked up by "<config.workload> | <launch>": each
    # workload whose dominant kernel was counted must keep the name the bench
    # line gives it, or its traffic would silently read null.
    kernels = json.loads((Path(bench.__file__).parent / "profiles" / "traffic.json").read_text())["kernels"]
    workloads = {key.split(" | ")[0] for key in kernels}
    assert bench.mlp_workload(8192) in workloads
    assert bench.BF16_WORKLOAD in workloads
    # At least the algorithmic bytes: A and B in bf16 (2 x 128 MiB) read, C in fp32 (256 MiB) written.
    assert bench.measured_traffic(bench.BF16_WORKLOAD, "tensor_core_bf16") >= 2 ** 29
    assert bench.measured_traffic(bench.BF16_WORKLOAD, "no such kernel") is None
