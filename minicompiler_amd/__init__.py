"""Python binding of libminicompiler_hip.so, the MI355X (gfx950) backend of
the minicompiler ML-graph compiler.

A thin ctypes layer over the C ABI in include/minicompiler_hip.h, shaped like
the reference's own ctypes harness (bench/torch_compare.py over
bench/capi.cpp): compile a .mcg graph, upload inputs, enqueue on a stream,
download outputs; plus the GEMM operator, the kernel generator and device
memory, stream and event calls. The compute path is the HIP library only:
if the library is not built, every call raises LibraryMissing (there is no
CPU fallback).

Do not use this binding in a process that also uses PyTorch's GPU runtime:
both would load a libamdhip64.so.7.
"""

from __future__ import annotations

import ctypes
import json
import os
from pathlib import Path
from typing import Iterable, Sequence

import numpy as np

PACKAGE_DIR = Path(__file__).resolve().parent
LIBRARY_PATH = PACKAGE_DIR / "lib" / "libminicompiler_hip.so"
GRAPHS_DIR = PACKAGE_DIR / "graphs"

# MatmulKernel values (include/minicompiler/hip/hip_backend.hpp).
MATMUL_KERNELS = ["auto", "naive", "tiled", "register_tiled_128", "register_tiled_64", "vectorized",
                  "double_buffered", "split_k", "tensor_core_tf32", "tensor_core_bf16", "tensor_core_f16"]
DTYPE_BF16 = 1
DTYPE_F16 = 2


class LibraryMissing(RuntimeError):
    pass


class MinicompilerError(RuntimeError):
    pass


class HipError(RuntimeError):
    def __init__(self, call: str, code: int):
        super().__init__(f"{call}: {error_string(code)} ({code})")
        self.code = code


_lib: ctypes.CDLL | None = None

_c = ctypes
_vp, _cp, _i, _ll, _sz, _d, _f = _c.c_void_p, _c.c_char_p, _c.c_int, _c.c_longlong, _c.c_size_t, _c.c_double, _c.c_float
_fp = _c.POINTER(_c.c_float)

_SIGNATURES = {
    "mc_compile": (_vp, [_cp, _cp, _cp, _cp, _cp, _i]),
    "mc_compile_source": (_vp, [_cp, _cp, _cp, _cp, _cp, _cp, _i]),
    "mc_num_inputs": (_i, [_vp]),
    "mc_num_outputs": (_i, [_vp]),
    "mc_output_elements": (_ll, [_vp, _i]),
    "mc_input_elements": (_ll, [_vp, _i]),
    "mc_run": (_i, [_vp, _c.POINTER(_vp), _c.POINTER(_vp)]),
    "mc_upload": (_i, [_vp, _c.POINTER(_vp)]),
    "mc_enqueue": (_i, [_vp, _vp]),
    "mc_download": (_i, [_vp, _c.POINTER(_vp)]),
    "mc_kernel_launches": (_i, [_vp]),
    "mc_matmul_kernels": (_i, [_vp, _cp, _i]),
    "mc_gpu_sm_clock_mhz": (_d, []),
    "mc_gpu_clock_sample": (_i, [_c.POINTER(_d), _c.POINTER(_c.c_ulonglong)]),
    "mc_gpu_device_json": (_i, [_c.POINTER(_d), _i, _cp, _i]),
    "mc_release": (None, [_vp]),
    "mc_last_error": (_i, [_cp, _i]),
    "mc_bind_inputs": (_i, [_vp, _c.POINTER(_vp)]),
    "mc_bind_outputs": (_i, [_vp, _c.POINTER(_vp)]),
    "mc_input_device_ptr": (_vp, [_vp, _i]),
    "mc_output_device_ptr": (_vp, [_vp, _i]),
    "mc_stream": (_vp, [_vp]),
    "mc_synchronize": (_i, [_vp]),
    "mc_jit_compile_ms": (_d, [_vp]),
    "mc_intermediate_bytes": (_ll, [_vp]),
    "mc_arena_bytes": (_ll, [_vp]),
    "mc_profile_start": (_i, [_vp, _i]),
    "mc_enqueue_profiled": (_i, [_vp, _vp]),
    "mc_enqueue_launch": (_i, [_vp, _i, _vp]),
    "mc_enqueue_steps": (_i, [_vp, _i, _i, _i, _c.POINTER(_vp), _c.POINTER(_vp), _vp, _c.POINTER(_d)]),
    "mc_launch_nodes": (_i, [_vp, _cp, _i]),
    "mc_profile_read": (_i, [_vp, _fp, _i]),
    "mc_launch_names": (_i, [_vp, _cp, _i]),
    "mc_fill_uniform": (None, [_fp, _sz, _c.c_ulonglong, _f, _f]),
    "mc_fill_normal": (None, [_fp, _sz, _c.c_ulonglong, _d, _d]),
    "mc_graph_json": (_i, [_vp, _cp, _i]),
    "mc_constant_values": (_i, [_vp, _i, _fp, _ll]),
    "mc_stage_stats_json": (_i, [_vp, _cp, _i]),
    "mc_plan_json": (_i, [_vp, _i, _cp, _i]),
    "mc_kernel_sources": (_i, [_vp, _cp, _i]),
    "mc_print_graph": (_i, [_vp, _cp, _i]),
    "mc_generate_elementwise_kernel": (_i, [_cp, _cp, _cp, _i, _i, _c.POINTER(_i), _cp, _i]),
    "mc_compile_kernel_source": (_i, [_cp, _cp, _cp, _i]),
    "mc_generate_gemm_epilogue_kernel": (_i, [_cp, _i, _cp, _cp, _i, _cp, _cp, _i]),
    "mc_launch_matmul": (_i, [_i, _vp, _vp, _vp, _i, _i, _i, _vp, _i, _vp]),
    "mc_launch_matmul_cfg": (_i, [_i, _vp, _vp, _vp, _i, _i, _i, _vp, _i, _vp, _i]),
    "mc_launch_matmul_lowp": (_i, [_i, _i, _vp, _vp, _vp, _i, _i, _i, _vp, _i, _vp]),
    "mc_launch_matmul_noalloc": (_i, [_i, _vp, _vp, _vp, _i, _i, _i, _vp, _i]),
    "mc_noalloc_scratch_bytes": (_c.c_ulonglong, []),
    "mc_convert_f32": (_i, [_i, _vp, _vp, _sz, _vp]),
    "mc_packed_a16_bytes": (_ll, [_i, _i]),
    "mc_pack_a16": (_i, [_vp, _vp, _i, _i, _vp]),
    "mc_convert_pack_a_f32": (_i, [_i, _vp, _vp, _i, _i, _vp]),
    "mc_launch_matmul_lowp_packed": (_i, [_i, _i, _vp, _vp, _vp, _i, _i, _i, _vp]),
    "mc_sum_split_partials": (_i, [_vp, _vp, _sz, _i, _vp]),
    "mc_split_k_splits": (_i, [_i, _i, _i, _i, _i]),
    "mc_matmul_splits": (_i, [_i, _i, _i, _i, _i]),
    "mc_matmul_workspace_bytes": (_ll, [_i, _i, _i, _i]),
    "mc_matmul_k_ranges": (_i, [_i, _i, _i, _i, _i]),
    "mc_resolve_matmul_kernel": (_i, [_i, _i, _i, _i, _i]),
    "mc_matmul_kernel_name": (_cp, [_i]),
    "mc_matmul_kernel_from_name": (_i, [_cp]),
    "mc_matmul_supported": (_i, [_i]),
    "mc_device_count": (_i, []),
    "mc_device_malloc": (_i, [_c.POINTER(_vp), _sz]),
    "mc_device_free": (_i, [_vp]),
    "mc_memcpy_htod": (_i, [_vp, _vp, _sz]),
    "mc_memcpy_dtoh": (_i, [_vp, _vp, _sz]),
    "mc_memcpy_dtod_async": (_i, [_vp, _vp, _sz, _vp]),
    "mc_memset": (_i, [_vp, _i, _sz]),
    "mc_device_synchronize": (_i, []),
    "mc_stream_create": (_i, [_c.POINTER(_vp)]),
    "mc_stream_destroy": (_i, [_vp]),
    "mc_stream_synchronize": (_i, [_vp]),
    "mc_event_create": (_i, [_c.POINTER(_vp)]),
    "mc_event_destroy": (_i, [_vp]),
    "mc_event_record": (_i, [_vp, _vp]),
    "mc_event_elapsed_ms": (_i, [_vp, _vp, _c.POINTER(_f)]),
    "mc_stream_begin_capture": (_i, [_vp]),
    "mc_stream_end_capture": (_i, [_vp, _c.POINTER(_vp)]),
    "mc_graph_launch": (_i, [_vp, _vp]),
    "mc_graph_destroy": (_i, [_vp]),
    "mc_error_string": (_cp, [_i]),
}


def library() -> ctypes.CDLL:
    """The loaded backend library; raises LibraryMissing if it is not built."""
    global _lib
    if _lib is None:
        path = Path(os.environ.get("MINICOMPILER_HIP_LIBRARY", LIBRARY_PATH))
        if not path.exists():
            raise LibraryMissing(f"{path} is not built: run `python -m minicompiler_amd.build` "
                                 "(or __graft_entry__.build())")
        lib = ctypes.CDLL(str(path))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def exported_symbols() -> list[str]:
    return list(_SIGNATURES)


def _text_call(fn, *args) -> str:
    """Calls a text-out function twice: once for the size, once for the text."""
    n = fn(*args, None, 0)
    if n < 0:
        raise MinicompilerError(last_error())
    buf = ctypes.create_string_buffer(n + 1)
    fn(*args, buf, n + 1)
    return buf.value.decode()


def last_error() -> str:
    return _text_call(library().mc_last_error)


def error_string(code: int) -> str:
    return library().mc_error_string(code).decode()


def _check(rc: int, call: str) -> None:
    if rc != 0:
        raise HipError(call, rc)


def _check_graph(rc: int, call: str) -> None:
    if rc != 0:
        raise MinicompilerError(f"{call}: {last_error()}")


# ---------------------------------------------------------------- device


def device_count() -> int:
    return library().mc_device_count()


def device_json(clocks: Sequence[float] = ()) -> dict:
    arr = (ctypes.c_double * max(1, len(clocks)))(*clocks)
    buf = ctypes.create_string_buffer(8192)
    rc = library().mc_gpu_device_json(arr if clocks else None, len(clocks), buf, len(buf))
    if rc != 0:
        raise MinicompilerError("no HIP device" if rc == 1 else "device JSON too long")
    return json.loads(buf.value.decode())


def synchronize() -> None:
    _check(library().mc_device_synchronize(), "hipDeviceSynchronize")


class DeviceBuffer:
    """A hipMalloc'd region of `nbytes` bytes."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        _check(library().mc_device_malloc(ctypes.byref(p), max(self.nbytes, 4)), "hipMalloc")
        self.ptr = p.value

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        buf = cls(a.nbytes)
        buf.upload(a)
        return buf

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes, "array larger than the buffer"
        _check(library().mc_memcpy_htod(self.ptr, a.ctypes.data, a.nbytes), "hipMemcpy H2D")

    def download(self, dtype=np.float32, count: int | None = None) -> np.ndarray:
        dtype = np.dtype(dtype)
        count = self.nbytes // dtype.itemsize if count is None else count
        out = np.empty(count, dtype=dtype)
        _check(library().mc_memcpy_dtoh(out.ctypes.data, self.ptr, out.nbytes), "hipMemcpy D2H")
        return out

    def fill_bytes(self, value: int) -> None:
        _check(library().mc_memset(self.ptr, value, self.nbytes), "hipMemset")

    def free(self) -> None:
        if self.ptr:
            library().mc_device_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Stream:
    def __init__(self):
        p = ctypes.c_void_p()
        _check(library().mc_stream_create(ctypes.byref(p)), "hipStreamCreate")
        self.handle = p.value

    def synchronize(self) -> None:
        _check(library().mc_stream_synchronize(self.handle), "hipStreamSynchronize")

    def __del__(self):
        try:
            if self.handle:
                library().mc_stream_destroy(self.handle)
        except Exception:
            pass


class Event:
    def __init__(self):
        p = ctypes.c_void_p()
        _check(library().mc_event_create(ctypes.byref(p)), "hipEventCreate")
        self.handle = p.value

    def record(self, stream=None) -> None:
        s = stream.handle if isinstance(stream, Stream) else stream
        _check(library().mc_event_record(self.handle, s), "hipEventRecord")

    def elapsed_ms(self, later: "Event") -> float:
        ms = ctypes.c_float()
        _check(library().mc_event_elapsed_ms(self.handle, later.handle, ctypes.byref(ms)), "hipEventElapsedTime")
        return float(ms.value)

    def __del__(self):
        try:
            if self.handle:
                library().mc_event_destroy(self.handle)
        except Exception:
            pass


class CapturedGraph:
    """The launches `record(stream)` enqueues on `stream`, captured into a HIP
    graph (nothing runs while recording); launch() replays them."""

    def __init__(self, stream: "Stream", record):
        lib = library()
        _check(lib.mc_stream_begin_capture(stream.handle), "hipStreamBeginCapture")
        try:
            record(stream)
        finally:
            p = ctypes.c_void_p()
            rc = lib.mc_stream_end_capture(stream.handle, ctypes.byref(p))
        _check(rc, "hipStreamEndCapture / hipGraphInstantiate")
        self.handle = p.value
        self.stream = stream

    def launch(self) -> None:
        _check(library().mc_graph_launch(self.handle, self.stream.handle), "hipGraphLaunch")

    def __del__(self):
        try:
            if self.handle:
                library().mc_graph_destroy(self.handle)
        except Exception:
            pass


def gpu_clock_mhz() -> float:
    """The engine clock of device 0 (AMD SMI's snapshot, refreshed about once
    a second), 0 if unreadable."""
    return float(library().mc_gpu_sm_clock_mhz())


def gpu_clock_sample() -> tuple[float, int]:
    """(MHz, firmware timestamp in ns of the snapshot) for device 0; (0, 0)
    if unreadable. Reads with the same timestamp are one snapshot."""
    mhz, stamp = ctypes.c_double(), ctypes.c_ulonglong()
    if library().mc_gpu_clock_sample(ctypes.byref(mhz), ctypes.byref(stamp)) != 0:
        return 0.0, 0
    return float(mhz.value), int(stamp.value)


def _stream_handle(stream):
    return stream.handle if isinstance(stream, Stream) else stream


def uniform(count: int, seed: int, lo: float, hi: float) -> np.ndarray:
    """The library's fill_uniform (the reference's seeded generator)."""
    out = np.empty(count, dtype=np.float32)
    library().mc_fill_uniform(out.ctypes.data_as(_fp), count, seed, lo, hi)
    return out


def normal(count: int, seed: int, mean: float, std: float) -> np.ndarray:
    out = np.empty(count, dtype=np.float32)
    library().mc_fill_normal(out.ctypes.data_as(_fp), count, seed, mean, std)
    return out


# ---------------------------------------------------------------- graphs


def _ptr_array(ptrs: Iterable) -> ctypes.Array:
    ptrs = list(ptrs)
    return (ctypes.c_void_p * max(1, len(ptrs)))(*ptrs)


def _dims_text(dims) -> str:
    if not dims:
        return ""
    if isinstance(dims, str):
        return dims
    return ",".join(f"{k}={v}" for k, v in dims.items())


def _options_text(options) -> str:
    if not options:
        return ""
    if isinstance(options, str):
        return options
    return ",".join(f"{k}={int(v) if isinstance(v, bool) else v}" for k, v in options.items())


class Compiled:
    """A graph run through the pass pipeline and compiled for `backend`
    ("hip", or "none" for the passes only, which needs no device)."""

    def __init__(self, text: str | None = None, *, path: str | os.PathLike | None = None, dims=None,
                 passes: str = "default", backend: str = "hip", options=None):
        lib = library()
        err = ctypes.create_string_buffer(1 << 16)
        if path is not None:
            if options:
                text = Path(path).read_text()
            else:
                self._h = lib.mc_compile(str(path).encode(), _dims_text(dims).encode(), passes.encode(),
                                         backend.encode(), err, len(err))
        if path is None or options:
            self._h = lib.mc_compile_source(text.encode(), _dims_text(dims).encode(), passes.encode(),
                                            backend.encode(), _options_text(options).encode(), err, len(err))
        if not self._h:
            raise MinicompilerError(err.value.decode())
        self.backend = backend
        self.num_inputs = lib.mc_num_inputs(self._h)
        self.num_outputs = lib.mc_num_outputs(self._h)
        self.input_sizes = [lib.mc_input_elements(self._h, k) for k in range(self.num_inputs)]
        self.output_sizes = [lib.mc_output_elements(self._h, k) for k in range(self.num_outputs)]
        self._graph = None

    # -- running
    def _inputs(self, inputs: Sequence[np.ndarray]) -> tuple[list[np.ndarray], ctypes.Array]:
        if len(inputs) != self.num_inputs:
            raise ValueError(f"expected {self.num_inputs} inputs, got {len(inputs)}")
        arrs = []
        for k, a in enumerate(inputs):
            a = np.ascontiguousarray(a, dtype=np.float32)
            if a.size != self.input_sizes[k]:
                raise ValueError(f"input {k} has {a.size} elements, expected {self.input_sizes[k]}")
            arrs.append(a)
        return arrs, _ptr_array(a.ctypes.data for a in arrs)

    def _outputs(self) -> tuple[list[np.ndarray], ctypes.Array]:
        outs = [np.full(n, np.nan, dtype=np.float32) for n in self.output_sizes]
        return outs, _ptr_array(o.ctypes.data for o in outs)

    def run(self, inputs: Sequence[np.ndarray]) -> list[np.ndarray]:
        arrs, ip = self._inputs(inputs)
        outs, op = self._outputs()
        _check_graph(library().mc_run(self._h, ip, op), "mc_run")
        return outs

    def upload(self, inputs: Sequence[np.ndarray]) -> None:
        arrs, ip = self._inputs(inputs)
        _check_graph(library().mc_upload(self._h, ip), "mc_upload")

    def enqueue(self, stream=None) -> None:
        _check_graph(library().mc_enqueue(self._h, _stream_handle(stream)), "mc_enqueue")

    def download(self) -> list[np.ndarray]:
        outs, op = self._outputs()
        _check_graph(library().mc_download(self._h, op), "mc_download")
        return outs

    def synchronize(self) -> None:
        _check_graph(library().mc_synchronize(self._h), "mc_synchronize")

    def profile_start(self, steps: int) -> None:
        _check_graph(library().mc_profile_start(self._h, steps), "mc_profile_start")

    def enqueue_launch(self, j: int, stream=None) -> None:
        _check_graph(library().mc_enqueue_launch(self._h, j, _stream_handle(stream)), "mc_enqueue_launch")

    def enqueue_steps(self, steps: int, launch: int = -1, sets=None, stream=None) -> float:
        """`steps` enqueues in one library call (launch -1: the whole step,
        else launch `launch` alone), binding buffer set i % len(sets) before
        step i when `sets` (a list of (input_ptrs, output_ptrs)) is given.
        Returns the host microseconds per step of the loop."""
        ni, no = self.num_inputs, self.num_outputs
        n = len(sets) if sets else 0
        ip = (ctypes.c_void_p * max(1, n * ni))(*[p for ins, _ in (sets or []) for p in ins])
        op = (ctypes.c_void_p * max(1, n * no))(*[p for _, outs in (sets or []) for p in outs])
        us = ctypes.c_double()
        _check_graph(library().mc_enqueue_steps(self._h, launch, steps, n, ip, op, _stream_handle(stream),
                                                ctypes.byref(us)), "mc_enqueue_steps")
        return float(us.value)

    def enqueue_profiled(self, stream=None) -> None:
        _check_graph(library().mc_enqueue_profiled(self._h, _stream_handle(stream)), "mc_enqueue_profiled")

    def profile_read(self) -> np.ndarray:
        """steps x launches durations in ms of the profiled enqueues."""
        n = library().mc_profile_read(self._h, None, 0)
        if n < 0:
            raise MinicompilerError(last_error())
        out = np.empty(max(n, 1), dtype=np.float32)
        library().mc_profile_read(self._h, out.ctypes.data_as(_fp), n)
        launches = self.kernel_launches
        return out[:n].reshape(-1, launches) if launches else out[:0]

    @property
    def launch_names(self) -> list[str]:
        return [s for s in _text_call(library().mc_launch_names, self._h).split("\n") if s]

    def bind_inputs(self, ptrs: Sequence[int | None]) -> None:
        _check_graph(library().mc_bind_inputs(self._h, _ptr_array(ptrs)), "mc_bind_inputs")

    def bind_outputs(self, ptrs: Sequence[int | None]) -> None:
        _check_graph(library().mc_bind_outputs(self._h, _ptr_array(ptrs)), "mc_bind_outputs")

    def input_ptr(self, k: int) -> int:
        return library().mc_input_device_ptr(self._h, k)

    def output_ptr(self, k: int) -> int:
        return library().mc_output_device_ptr(self._h, k)

    @property
    def stream(self) -> int:
        return library().mc_stream(self._h)

    # -- reports
    @property
    def kernel_launches(self) -> int:
        return library().mc_kernel_launches(self._h)

    @property
    def matmul_kernels(self) -> list[str]:
        # Returns 0 or 1 like the reference's (bench/capi.cpp:184-202), not a length.
        buf = ctypes.create_string_buffer(64 * max(1, self.kernel_launches) + 64)
        if library().mc_matmul_kernels(self._h, buf, len(buf)) != 0:
            raise MinicompilerError(last_error())
        return [s for s in buf.value.decode().split(",") if s]

    @property
    def launch_nodes(self) -> list[list[int]]:
        """Graph node ids each launch computes (a fused matmul: matmul, group)."""
        text = _text_call(library().mc_launch_nodes, self._h)
        return [[int(x) for x in part.split(",")] for part in text.split(";") if part]

    @property
    def kernel_sources(self) -> list[str]:
        text = _text_call(library().mc_kernel_sources, self._h)
        return [s for s in text.split("//----\n") if s] if text else []

    @property
    def jit_compile_ms(self) -> float:
        return library().mc_jit_compile_ms(self._h)

    @property
    def intermediate_bytes(self) -> int:
        return library().mc_intermediate_bytes(self._h)

    @property
    def arena_bytes(self) -> int:
        return library().mc_arena_bytes(self._h)

    def graph(self) -> dict:
        if self._graph is None:
            self._graph = json.loads(_text_call(library().mc_graph_json, self._h))
        return self._graph

    def constant(self, node: int) -> np.ndarray:
        g = self.graph()
        count = int(np.prod(g["nodes"][node]["shape"], dtype=np.int64))
        out = np.empty(count, dtype=np.float32)
        _check_graph(library().mc_constant_values(self._h, node, out.ctypes.data_as(_fp), count), "mc_constant_values")
        return out

    def stage_stats(self) -> list[dict]:
        return json.loads(_text_call(library().mc_stage_stats_json, self._h))

    def plan(self, pool_outputs: bool = True) -> dict:
        return json.loads(_text_call(library().mc_plan_json, self._h, 1 if pool_outputs else 0))

    def print_graph(self) -> str:
        return _text_call(library().mc_print_graph, self._h)

    def close(self) -> None:
        if getattr(self, "_h", None):
            library().mc_release(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def graph_path(name: str) -> Path:
    return GRAPHS_DIR / f"{name}.mcg"


# ---------------------------------------------------------------- GEMM operator


def matmul_kernel_id(name: str) -> int:
    k = library().mc_matmul_kernel_from_name(name.encode())
    if k < 0:
        raise ValueError(f"unknown matmul kernel {name!r}")
    return k


def matmul_kernel_name(kernel: int) -> str:
    return library().mc_matmul_kernel_name(kernel).decode()


def launch_matmul(kernel: int | str, a: int, b: int, c: int, m: int, n: int, k: int, stream=None, splits: int = 1,
                  workspace: int | None = None) -> None:
    kid = matmul_kernel_id(kernel) if isinstance(kernel, str) else kernel
    _check(library().mc_launch_matmul(kid, a, b, c, m, n, k, _stream_handle(stream), splits, workspace),
           f"launch_matmul({matmul_kernel_name(kid)})")


def launch_matmul_noalloc(kernel: int | str, a: int, b: int, c: int, m: int, n: int, k: int, stream=None,
                          splits: int = 1) -> None:
    """launch_matmul with the split-K partials in the library's per-GPU
    scratch array (noalloc_scratch_bytes()); allocates nothing. Calls that
    overlap on one GPU race on the array."""
    kid = matmul_kernel_id(kernel) if isinstance(kernel, str) else kernel
    rc = library().mc_launch_matmul_noalloc(kid, a, b, c, m, n, k, _stream_handle(stream), splits)
    if rc != 0:
        raise HipError(f"launch_matmul_noalloc({matmul_kernel_name(kid)}): {last_error()}", rc)


def noalloc_scratch_bytes() -> int:
    return int(library().mc_noalloc_scratch_bytes())


RING_CONFIGS = {"auto": 0, "wide": 1, "mid": 2, "big": 3, "thin": 4, "narrow": 5, "wide8": 6}


def launch_matmul_cfg(kernel: int | str, a: int, b: int, c: int, m: int, n: int, k: int, stream=None,
                      splits: int = 1, workspace: int | None = None, ring: int | str = "auto") -> None:
    """launch_matmul with the FP32 ring configuration forced (RING_CONFIGS)."""
    kid = matmul_kernel_id(kernel) if isinstance(kernel, str) else kernel
    cfg = RING_CONFIGS[ring] if isinstance(ring, str) else ring
    _check(library().mc_launch_matmul_cfg(kid, a, b, c, m, n, k, _stream_handle(stream), splits, workspace, cfg),
           f"launch_matmul_cfg({matmul_kernel_name(kid)}, ring {ring})")


def launch_matmul_lowp(kernel: int | str, dtype: int, a: int, b: int, c: int, m: int, n: int, k: int, stream=None,
                       splits: int = 1, workspace: int | None = None) -> None:
    kid = matmul_kernel_id(kernel) if isinstance(kernel, str) else kernel
    _check(library().mc_launch_matmul_lowp(kid, dtype, a, b, c, m, n, k, _stream_handle(stream), splits, workspace),
           f"launch_matmul_lowp({matmul_kernel_name(kid)})")


def memcpy_dtod_async(dst: int, src: int, nbytes: int, stream=None) -> None:
    """The HIP runtime's device-to-device copy (hipMemcpyAsync), enqueued on `stream`."""
    _check(library().mc_memcpy_dtod_async(dst, src, nbytes, _stream_handle(stream)), "hipMemcpyAsync D2D")


def convert_f32(dtype: int, src: int, dst: int, count: int, stream=None) -> None:
    _check(library().mc_convert_f32(dtype, src, dst, count, _stream_handle(stream)), "convert_f32")


def packed_a16_bytes(m: int, k: int) -> int:
    """Bytes of packed A (mc_pack_a16's layout) for an m x k operand."""
    return int(library().mc_packed_a16_bytes(m, k))


def pack_a16(src: int, dst: int, m: int, k: int, stream=None) -> None:
    """16-bit row-major A [m, k] to packed A."""
    _check(library().mc_pack_a16(src, dst, m, k, _stream_handle(stream)), "pack_a16")


def convert_pack_a_f32(dtype: int, src: int, dst: int, m: int, k: int, stream=None) -> None:
    """fp32 row-major A [m, k] rounded to bf16 (dtype 1) / fp16 (dtype 2) and packed."""
    _check(library().mc_convert_pack_a_f32(dtype, src, dst, m, k, _stream_handle(stream)), "convert_pack_a_f32")


def launch_matmul_lowp_packed(kernel: int | str, dtype: int, a_packed: int, b: int, c: int, m: int, n: int, k: int,
                              stream=None) -> None:
    """The bf16/fp16 product on packed A and row-major 16-bit B."""
    kid = matmul_kernel_id(kernel) if isinstance(kernel, str) else kernel
    _check(library().mc_launch_matmul_lowp_packed(kid, dtype, a_packed, b, c, m, n, k, _stream_handle(stream)),
           f"launch_matmul_lowp_packed({matmul_kernel_name(kid)})")


def sum_split_partials(partial: int, c: int, count: int, splits: int, stream=None) -> None:
    """c[i] = partial[0][i] + ... + partial[splits-1][i], added in split order."""
    _check(library().mc_sum_split_partials(partial, c, count, splits, _stream_handle(stream)), "sum_split_partials")


def split_k_splits(m: int, n: int, k: int, cu_count: int, blocks_per_cu: int = 2) -> int:
    return library().mc_split_k_splits(m, n, k, cu_count, blocks_per_cu)


def matmul_splits(kernel: int | str, m: int, n: int, k: int, cu_count: int) -> int:
    kid = matmul_kernel_id(kernel) if isinstance(kernel, str) else kernel
    return library().mc_matmul_splits(kid, m, n, k, cu_count)


def matmul_k_ranges(kernel: int | str, m: int, n: int, k: int, splits: int) -> int:
    """The K ranges launch_matmul runs given `splits` (an upper bound: the
    narrow-tile body of split_k may run fewer)."""
    return int(library().mc_matmul_k_ranges(matmul_kernel_id(kernel), m, n, k, splits))


def matmul_workspace_bytes(kernel: int | str, m: int, n: int, splits: int) -> int:
    kid = matmul_kernel_id(kernel) if isinstance(kernel, str) else kernel
    return library().mc_matmul_workspace_bytes(kid, m, n, splits)


def resolve_matmul_kernel(kernel: int | str, m: int, n: int, k: int, cu_count: int) -> str:
    kid = matmul_kernel_id(kernel) if isinstance(kernel, str) else kernel
    return matmul_kernel_name(library().mc_resolve_matmul_kernel(kid, m, n, k, cu_count))


def matmul_supported(kernel: int | str) -> bool:
    kid = matmul_kernel_id(kernel) if isinstance(kernel, str) else kernel
    return bool(library().mc_matmul_supported(kid))


# ---------------------------------------------------------------- generator


def generate_elementwise_kernel(program: str, input_shapes: Sequence[Sequence[int]], out_shape: Sequence[int],
                                allow_vectorize: bool = True, items_per_lane: int = 0) -> tuple[str, bool]:
    shapes = ";".join("[" + ",".join(str(d) for d in s) + "]" for s in input_shapes)
    out = "[" + ",".join(str(d) for d in out_shape) + "]"
    vec = ctypes.c_int(0)
    lib = library()
    n = lib.mc_generate_elementwise_kernel(program.encode(), shapes.encode(), out.encode(), int(allow_vectorize),
                                           items_per_lane, ctypes.byref(vec), None, 0)
    if n < 0:
        raise MinicompilerError(last_error())
    buf = ctypes.create_string_buffer(n + 1)
    lib.mc_generate_elementwise_kernel(program.encode(), shapes.encode(), out.encode(), int(allow_vectorize),
                                       items_per_lane, ctypes.byref(vec), buf, n + 1)
    return buf.value.decode(), bool(vec.value)


def generate_gemm_epilogue_kernel(program: str, acc_input: int, input_shapes: Sequence[Sequence[int]],
                                  out_shape: Sequence[int], vectorized_operands: bool = True,
                                  body: str = "two_stage") -> str:
    shapes = ";".join("[" + ",".join(str(d) for d in s) + "]" for s in input_shapes)
    out = "[" + ",".join(str(d) for d in out_shape) + "]"
    args = (program.encode(), acc_input, shapes.encode(), out.encode(), int(vectorized_operands), body.encode())
    return _text_call(library().mc_generate_gemm_epilogue_kernel, *args)


def compile_kernel_source(source: str, arch: str = "gfx950") -> tuple[bool, str]:
    log = ctypes.create_string_buffer(1 << 16)
    rc = library().mc_compile_kernel_source(source.encode(), arch.encode(), log, len(log))
    return rc == 0, log.value.decode()
