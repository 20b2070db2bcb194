"""Packed A for the bf16/fp16 256x256-tile kernel, through the C ABI: the
layout the packing kernels write (against a numpy reshape of the padded
operand, not the kernels' index arithmetic), rounding while packing (against
rounding then packing), and the product on packed A (the same bits as on
row-major A, with every element of C written and nothing past it). The
reference has no counterpart: its tensor-core kernel stages row-major fp32
(src/cuda/matmul_tensor_core.cu:96-297); these results are pinned to this
library's own row-major kernel, itself checked against float64 in
test_gpu_mfma.py."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GUARD = 4096


def numpy_packed(a16: np.ndarray, m: int, k: int) -> np.ndarray:
    # Rows padded to whole 256-row bands with zeros; row = 256 band + 16 rb +
    # r16 and k = 32 s + 8 c + e, stored in the order (band, s, rb, c, r16, e).
    bands = (m + 255) // 256
    pad = np.zeros((bands * 256, k), np.uint16)
    pad[:m] = a16.reshape(m, k)
    return pad.reshape(bands, 16, 16, k // 32, 4, 8).transpose(0, 3, 1, 4, 2, 5).reshape(-1)


def rand16(seed: int, count: int) -> np.ndarray:
    # Finite bf16 / fp16 bit patterns of moderate size (exponent bits kept
    # away from inf / NaN), so a product of them is a plain float.
    rng = np.random.default_rng(seed)
    return (rng.integers(0, 1 << 16, count, dtype=np.uint32) & 0xBFFF).astype(np.uint16) | 0x2000


@pytest.mark.parametrize("m,k", [(256, 64), (300, 128), (1, 64), (513, 192)])
def test_pack_a16_writes_the_packed_layout(device, mc, m, k):
    print(f"case pack {m}x{k}", flush=True)
    a16 = rand16(1, m * k)
    nbytes = mc.packed_a16_bytes(m, k)
    assert nbytes == ((m + 255) // 256) * 256 * k * 2
    src = mc.DeviceBuffer.from_array(a16)
    dst = mc.DeviceBuffer(nbytes)
    dst.fill_bytes(0xFF)
    mc.pack_a16(src.ptr, dst.ptr, m, k)
    mc.synchronize()
    got = dst.download(np.uint16, nbytes // 2)
    assert np.array_equal(got, numpy_packed(a16, m, k))
    # A source at a 2-byte offset takes the element-wise path: same packing.
    off = mc.DeviceBuffer(2 * m * k + 16)
    off.upload(np.concatenate([np.zeros(1, np.uint16), a16]))
    dst.fill_bytes(0xFF)
    mc.pack_a16(off.ptr + 2, dst.ptr, m, k)
    mc.synchronize()
    assert np.array_equal(dst.download(np.uint16, nbytes // 2), numpy_packed(a16, m, k))


@pytest.mark.parametrize("dtype", [1, 2])
@pytest.mark.parametrize("m,k", [(300, 128), (256, 1024), (513, 192)])  # 4, 32 and 6 K steps
def test_convert_pack_rounds_as_convert_f32(device, mc, oracle, dtype, m, k):
    print(f"case convert+pack dtype {dtype} {m}x{k}", flush=True)
    a32 = oracle.uniform(m * k, 3, -3.0, 3.0)
    a32[:7] = [np.inf, -np.inf, np.nan, 0.0, -0.0, 1e-40, 70000.0]
    src = mc.DeviceBuffer.from_array(a32)
    rounded = mc.DeviceBuffer(2 * m * k)
    mc.convert_f32(dtype, src.ptr, rounded.ptr, m * k)
    nbytes = mc.packed_a16_bytes(m, k)
    packed = mc.DeviceBuffer(nbytes)
    mc.convert_pack_a_f32(dtype, src.ptr, packed.ptr, m, k)
    mc.synchronize()
    want = numpy_packed(rounded.download(np.uint16, m * k), m, k)
    assert np.array_equal(packed.download(np.uint16, nbytes // 2), want)
    # fp32 A at a 4-byte offset: the element-wise loads, the same bits.
    off = mc.DeviceBuffer(4 * m * k + 16)
    off.upload(np.concatenate([np.zeros(1, np.float32), a32]))
    packed.fill_bytes(0xFF)
    mc.convert_pack_a_f32(dtype, off.ptr + 4, packed.ptr, m, k)
    mc.synchronize()
    assert np.array_equal(packed.download(np.uint16, nbytes // 2), want)


# (m, n, k): one tile; ragged M with every tile run as two 128-row halves (the
# second half of the last band past M); 272 tiles with the last 16 as halves
# and a ragged last band; ragged N; several rounds; the matrix edge inside C's 8-row by 32-column store pieces
# (M % 16 = 15 and 7, N % 32 = 24 and 16).
SHAPES = [(256, 256, 64), (300, 520, 256), (4300, 4096, 64), (1000, 1032, 512), (2048, 2048, 1024), (271, 280, 128),
          (263, 272, 192)]


@pytest.mark.parametrize("kernel,dtype", [("tensor_core_bf16", 1), ("tensor_core_f16", 2)])
@pytest.mark.parametrize("m,n,k", SHAPES)
def test_the_product_on_packed_a_equals_row_major_a_bit_for_bit(device, mc, kernel, dtype, m, n, k):
    print(f"case packed {kernel} {m}x{n}x{k}", flush=True)
    a16, b16 = rand16(11, m * k), rand16(12, k * n)
    da, db = mc.DeviceBuffer.from_array(a16), mc.DeviceBuffer.from_array(b16)
    dp = mc.DeviceBuffer(mc.packed_a16_bytes(m, k))
    mc.pack_a16(da.ptr, dp.ptr, m, k)
    outs = []
    for packed in (False, True):
        c = mc.DeviceBuffer.from_array(np.full(m * n + GUARD, np.nan, np.float32))
        if packed:
            mc.launch_matmul_lowp_packed(kernel, dtype, dp.ptr, db.ptr, c.ptr, m, n, k)
        else:
            mc.launch_matmul_lowp(kernel, dtype, da.ptr, db.ptr, c.ptr, m, n, k)
        mc.synchronize()
        out = c.download()
        assert np.all(np.isnan(out[m * n:])), "a write past the end of C"
        assert not np.any(np.isnan(out[:m * n])), "an element of C was not written"
        outs.append(out[:m * n])
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))


def test_packed_entry_points_refuse_what_the_kernel_cannot_take(device, mc):
    a = mc.DeviceBuffer(2 * 256 * 128 + 32)
    b = mc.DeviceBuffer(2 * 128 * 256 + 32)
    c = mc.DeviceBuffer(4 * 256 * 256 + 32)
    with pytest.raises(mc.HipError):
        mc.pack_a16(a.ptr, b.ptr, 256, 96)                      # K not a multiple of 64
    with pytest.raises(mc.HipError):
        mc.pack_a16(a.ptr, b.ptr + 8, 256, 64)                  # packed A not 16-byte aligned
    with pytest.raises(mc.HipError):
        mc.launch_matmul_lowp_packed("tensor_core_bf16", 1, a.ptr, b.ptr, c.ptr, 256, 252, 128)  # N % 8
    with pytest.raises(mc.HipError):
        mc.launch_matmul_lowp_packed("tensor_core_bf16", 1, a.ptr + 8, b.ptr, c.ptr, 256, 256, 128)  # alignment
    with pytest.raises(mc.HipError):
        mc.launch_matmul_lowp_packed("tensor_core_bf16", 2, a.ptr, b.ptr, c.ptr, 256, 256, 128)  # dtype mismatch
    mc.synchronize()
