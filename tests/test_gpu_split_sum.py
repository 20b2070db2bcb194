"""The split-K partial sum (mchip_sum_split_partials, the reference's
sum_split_partials at src/cuda/matmul_kernels.cu:340-350) against a numpy
left fold, bit for bit: c[i] = ((p0[i] + p1[i]) + p2[i]) + ... in float32.
The cases reach every lane width and load batch the launcher picks (float4
lanes with 4, 8 or 16 loads in flight; one float per lane with 8, 16, 32 or
64), batches that end past the last split, more splits than one batch, a
count that is not a multiple of 4, an unaligned pointer and one split. Rows
of -0.0 in every split check that the fold starts from split 0's value, and
the floats after C must stay untouched."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GUARD = 64  # floats after C, prefilled with NaN


def left_fold(p: np.ndarray) -> np.ndarray:
    s = p[0].copy()
    for z in range(1, p.shape[0]):
        s = s + p[z]  # float32 + float32, one rounding per add
    return s


# (count, splits): 262144 floats fill 256 CUs with float4 lanes; fewer use
# one float per lane.
CASES = [(262144, 5), (262144, 9), (262144, 20), (65536, 64), (65536, 8), (1001, 3), (1001, 17), (1001, 33),
         (262147, 65), (4096, 1), (262144, 2)]


@pytest.mark.parametrize("count,splits", CASES)
@pytest.mark.parametrize("offset", [0, 4], ids=["aligned", "c+4B"])
def test_split_sum_is_the_left_fold_bit_for_bit(device, mc, count, splits, offset):
    print(f"case split sum count={count} splits={splits} offset={offset}", flush=True)
    rng = np.random.default_rng(count * 131 + splits)
    p = (rng.uniform(-1.0, 1.0, (splits, count)) * 2.0 ** rng.integers(-20, 20, (splits, count))).astype(np.float32)
    p[:, :7] = np.float32(-0.0)
    expected = left_fold(p)
    dp = mc.DeviceBuffer.from_array(p.reshape(-1))
    dc = mc.DeviceBuffer(offset + 4 * (count + GUARD))
    dc.upload(np.full(offset // 4 + count + GUARD, np.nan, dtype=np.float32))
    mc.sum_split_partials(dp.ptr, dc.ptr + offset, count, splits)
    mc.synchronize()
    out = dc.download()[offset // 4:]
    assert np.all(np.isnan(out[count:])), "a write past the end of C"
    got = out[:count]
    assert np.array_equal(got.view(np.uint32), expected.view(np.uint32)), (
        f"{np.count_nonzero(got.view(np.uint32) != expected.view(np.uint32))} elements differ")
    assert np.all(np.signbit(got[:7])), "the fold must start from split 0's value (-0.0 + -0.0 = -0.0)"
