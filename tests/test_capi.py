"""The C ABI (include/minicompiler_hip.h) without a GPU: every declared
symbol is exported, errors come back as messages, and the pure-integer
matmul policy keeps the reference's known answers."""

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "minicompiler_hip.h"


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"MC_API[^;(]*?\b(mc_\w+)\s*\(", text)


def test_library_exports_every_declared_symbol(mc):
    names = declared_symbols()
    assert len(names) >= 50
    lib = mc.library()
    for n in names:
        assert hasattr(lib, n), n
    # The Python binding covers exactly the declared ABI.
    assert sorted(names) == sorted(mc.exported_symbols())
    out = subprocess.run(["nm", "-D", "--defined-only", str(mc.LIBRARY_PATH)], capture_output=True, text=True).stdout
    exported = set(re.findall(r" T (mc_\w+)", out))
    assert set(names) <= exported


def test_the_product_library_does_not_link_the_oracle(mc):
    out = subprocess.run(["readelf", "-d", str(mc.LIBRARY_PATH)], capture_output=True, text=True).stdout
    needed = re.findall(r"Shared library: \[(.*?)\]", out)
    assert not any("oracle" in n for n in needed), needed
    syms = subprocess.run(["nm", "-D", str(mc.LIBRARY_PATH)], capture_output=True, text=True).stdout
    assert "orc_" not in syms


def test_compile_errors_are_reported(mc):
    err = ctypes.create_string_buffer(4096)
    lib = mc.library()
    h = lib.mc_compile(b"/nonexistent.mcg", b"", b"default", b"hip", err, len(err))
    assert not h and b"cannot open" in err.value
    h = lib.mc_compile(str(mc.graph_path("gelu_chain")).encode(), b"M=x", b"default", b"hip", err, len(err))
    assert not h and b"bad dim" in err.value
    h = lib.mc_compile(str(mc.graph_path("gelu_chain")).encode(), b"", b"default", b"cpu", err, len(err))
    assert not h and b"not built into this library" in err.value
    h = lib.mc_compile(str(mc.graph_path("gelu_chain")).encode(), b"", b"default", b"tpu", err, len(err))
    assert not h and b"unknown backend 'tpu' (available: hip)" in err.value
    with pytest.raises(mc.MinicompilerError, match="unknown option"):
        mc.Compiled("input x : f32[2]\noutput x\n", backend="none", options="frob=1")
    with pytest.raises(mc.MinicompilerError, match="unknown matmul kernel"):
        mc.Compiled("input x : f32[2]\noutput x\n", backend="none", options="matmul=register_tiled_32")


def test_no_device_calls_fail_cleanly_on_the_cpu(mc):
    if mc.device_count() > 0:
        pytest.skip("a device is present")
    assert mc.library().mc_gpu_device_json(None, 0, None, 0) == 1
    assert mc.gpu_clock_sample() == (0.0, 0)  # mc_gpu_clock_sample returns 1 and zeroes both outputs
    assert mc.gpu_clock_mhz() == 0.0
    with pytest.raises(mc.MinicompilerError, match="no HIP device|no usable HIP device"):
        mc.Compiled("input x : f32[4]\ny = neg x\noutput y\n", backend="hip")
    c = mc.Compiled("input x : f32[4]\ny = neg x\noutput y\n", backend="none")
    assert c.kernel_launches == -1
    with pytest.raises(mc.MinicompilerError, match="no executable"):
        c.enqueue()


def test_split_k_rule_known_answers_on_30_cus(mc):
    # tests/test_cuda_backend.cpp:315-343, restated with the CU count as a parameter.
    s = mc.split_k_splits
    assert s(128, 512, 2048, 30, 2) == 7
    assert s(128, 1920, 2048, 30, 2) == 2
    assert s(128, 2048, 2048, 30, 2) == 3
    assert s(128, 2944, 2048, 30, 2) == 2
    assert s(128, 3072, 2048, 30, 2) == 1
    assert s(640, 640, 640, 30, 2) == 1
    assert s(1024, 1024, 1024, 30, 2) == 1
    assert s(128, 128, 200, 30, 2) == 3
    assert s(128, 128, 100, 30, 2) == 1
    assert s(128, 512, 2048, 30, 1) == 7
    assert s(128, 2048, 2048, 30, 1) == 1
    assert s(128, 1792, 2048, 30, 1) == 2
    for bpc in (1, 2):
        for tiles in range(1, 41):
            sp = s(128, 128 * tiles, 1 << 16, 30, bpc)
            if sp > 1:
                assert tiles * sp <= bpc * 30


def test_split_k_rule_on_256_cus(mc):
    s = mc.split_k_splits
    assert s(4096, 4096, 4096, 256, 2) == 1         # 1024 tiles fill the GPU
    assert s(1024, 1024, 1024, 256, 2) == 4         # 64 tiles: one block per CU
    assert s(256, 256, 16384, 256, 2) == 64         # 4 tiles
    assert s(16, 4096, 4096, 256, 2) == 8           # 32 tiles
    assert s(256, 512, 2048, 256, 2) == 32          # the MLP's second GEMM at B=256 (8 tiles)


def test_workspace_names_and_resolution(mc):
    wb = mc.matmul_workspace_bytes
    assert wb("split_k", 128, 512, 15) == 15 * 128 * 512 * 4
    assert wb("split_k", 128, 512, 1) == 0
    assert wb("double_buffered", 128, 512, 15) == 0
    assert wb("tensor_core_f16", 128, 512, 7) == 7 * 128 * 512 * 4
    assert wb("auto", 128, 512, 7) == 0
    for name in mc.MATMUL_KERNELS:
        assert mc.matmul_kernel_name(mc.matmul_kernel_id(name)) == name
    assert mc.library().mc_matmul_kernel_from_name(b"register_tiled_32") == -1
    r = mc.resolve_matmul_kernel
    # cuda_backend.cpp:358-373 known answers on 30 CUs.
    assert r("auto", 128, 512, 2048, 30) == "split_k"
    assert r("auto", 512, 512, 512, 30) == "split_k"
    assert r("auto", 640, 640, 640, 30) == "double_buffered"
    assert r("auto", 2048, 2048, 2048, 30) == "double_buffered"
    assert r("auto", 128, 128, 100, 30) == "double_buffered"
    assert r("auto", 640, 640, 640, 40) == "split_k"
    assert r("auto", 2 ** 31 - 1, 1, 1, 30) == "double_buffered"
    assert r("register_tiled_64", 4096, 4096, 4096, 30) == "register_tiled_64"
    assert r("naive", 1, 1, 1, 30) == "naive"
    assert not mc.matmul_supported("tensor_core_tf32")
    assert mc.matmul_supported("tensor_core_bf16") and mc.matmul_supported("tensor_core_f16")
