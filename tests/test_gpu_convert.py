"""fp32 -> bf16 / fp16 rounding on the GPU (mchip_convert_f32, the operand
rounding of the tensor-core matmuls, __float2bfloat16_rn / __float2half_rn at
src/cuda/matmul_tensor_core.cu:30-60 in the reference) against the oracle's
integer RNE (bf16) and numpy's IEEE conversion (fp16), bit for bit: special
values (signed zeros, infinities, NaN, subnormals, the largest finite values
and those that round past them, exact ties), random values over the whole
exponent range, counts with 0-3 elements past the last whole float4, and
both the aligned vector path and the unaligned scalar path. Bytes past the
last element stay untouched."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GUARD = 64  # bytes after the output, prefilled with 0xAB


def special_values() -> np.ndarray:
    bits = [0x00000000, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC00000, 0xFFC00001, 0x7F800001, 0x7FBFFFFF,
            0x00000001, 0x807FFFFF, 0x00800000, 0x7F7FFFFF, 0xFF7FFFFF,
            0x7F7F7FFF, 0x7F7F8000, 0x7F7F8001,  # bf16: below, at and above the tie before infinity
            0x3F808000, 0x3F818000, 0x3F808001, 0xBF808000,  # bf16 ties to even (down, up), above a tie, negative
            0x477FE000, 0x477FEFFF, 0x477FF000, 0x47800000,  # fp16: 65504, below / at the overflow tie, 65536
            0x33800000, 0x33000000, 0x33000001, 0x387FC000,  # fp16: smallest subnormal, half of it, just above, subnormal range
            0x3F801000, 0x3F803000]  # fp16 ties to even
    return np.array(bits, dtype=np.uint32).view(np.float32)


def inputs(count: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    x = (rng.uniform(-1.0, 1.0, count) * 2.0 ** rng.integers(-140, 128, count)).astype(np.float32)
    s = special_values()
    x[: min(count, s.size)] = s[: min(count, s.size)]
    return x


def expected_bits(x: np.ndarray, dtype: int) -> np.ndarray:
    from oracle import oracle

    r = oracle.round_bf16(x) if dtype == 1 else oracle.round_f16(x)
    if dtype == 1:
        return (r.view(np.uint32) >> 16).astype(np.uint16)
    return r.astype(np.float16).view(np.uint16)


@pytest.mark.parametrize("dtype", [1, 2], ids=["bf16", "fp16"])
@pytest.mark.parametrize("count", [0, 1, 3, 4, 5, 1027, 4099, 300_001])
@pytest.mark.parametrize("in_offset,out_offset", [(0, 0), (4, 0), (0, 2)], ids=["aligned", "in+4B", "out+2B"])
def test_rounding_matches_the_oracle_bit_for_bit(device, mc, dtype, count, in_offset, out_offset):
    print(f"case convert dtype={dtype} count={count} offsets={in_offset},{out_offset}", flush=True)
    x = inputs(count, 100 + count)
    src = mc.DeviceBuffer(in_offset + 4 * count + 16)
    src.upload(np.concatenate([np.zeros(in_offset // 4, np.float32), x]))
    dst = mc.DeviceBuffer(out_offset + 2 * count + GUARD)
    dst.fill_bytes(0xAB)
    mc.convert_f32(dtype, src.ptr + in_offset, dst.ptr + out_offset, count)
    mc.synchronize()
    raw = dst.download(np.uint8)
    got = raw[out_offset: out_offset + 2 * count].view(np.uint16)
    assert np.all(raw[:out_offset] == 0xAB) and np.all(raw[out_offset + 2 * count:] == 0xAB), "a write outside the output"
    want = expected_bits(x, dtype)
    nan_in = np.isnan(x)
    if dtype == 2:
        # fp16 NaN payloads are the hardware's; a NaN must stay a NaN.
        assert np.all(np.isnan(got[nan_in].view(np.float16)))
        got, want = got[~nan_in], want[~nan_in]
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, (f"{bad.size} of {got.size} differ; first at {bad[:4]}: got {got[bad[:4]]}, "
                           f"want {want[bad[:4]]}")
