"""The narrow-tile plan (mchip_f32_narrow_plan, host logic, no GPU): which
tile shape, how many K ranges and how deep each, for the split_k products the
bench and the MLP run, on 256 CUs. Shapes: 0 = 32x64, 1 = 16x64 with B
streamed (M <= 16), 2 = 16x64, 3 = 16x32, 4 = 64x64."""

import ctypes

import pytest

T32X64, T16X64_STREAM, T16X64, T16X32, T64X64 = 0, 1, 2, 3, 4


@pytest.fixture(scope="module")
def plan(mc):
    f = mc.library().mchip_f32_narrow_plan
    f.argtypes = [ctypes.c_int] * 6 + [ctypes.POINTER(ctypes.c_int)] * 3
    f.restype = ctypes.c_int

    def run(m, n, k, max_splits, cus=256, force=0):
        shape, splits, k_split = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        ok = f(m, n, k, max_splits, cus, force, ctypes.byref(shape), ctypes.byref(splits), ctypes.byref(k_split))
        return (shape.value, splits.value, k_split.value) if ok else None

    return run


@pytest.mark.parametrize("m,n,k,max_splits,want", [
    # Short K, unsplit: the first shape giving more than half the CUs a tile.
    (1024, 1024, 1024, 4, (T64X64, 1, 1024)),      # 256 tiles of 64x64
    (1024, 2048, 512, 2, (T64X64, 1, 512)),        # 512 tiles: 64x64 up to two per CU
    (1000, 1000, 528, 4, (T64X64, 1, 528)),        # ragged
    (256, 2048, 512, 8, (T32X64, 1, 512)),         # the MLP's GEMM1 at B=256
    (256, 512, 2048, 32, (T16X32, 1, 2048)),       # its GEMM2
    (512, 512, 512, 8, (T16X64, 1, 512)),
    (1024, 512, 2048, 8, (T32X64, 1, 2048)),       # the MLP's GEMM2 at B=1024
    # Long K: K ranges, 64x64 tiles where they need at most two.
    (16, 4096, 4096, 8, (T16X64_STREAM, 4, 1024)),
    (256, 256, 16384, 64, (T32X64, 8, 2048)),
    (128, 4096, 4096, 8, (T64X64, 2, 2048)),
    (1024, 1024, 4096, 4, (T64X64, 1, 4096)),
    (512, 512, 8192, 16, (T32X64, 2, 4096)),
])
def test_the_plan_for_the_bench_and_mlp_shapes(plan, m, n, k, max_splits, want):
    assert plan(m, n, k, max_splits) == want


def test_products_too_large_for_narrow_tiles_keep_the_ring(plan):
    assert plan(2048, 2048, 512, 2) is None       # 64x64 tiles four per CU
    assert plan(1024, 2048, 4096, 2) is None      # long K, 512 tiles of 64x64
    assert plan(8192, 512, 2048, 8) is None       # the MLP's GEMM2 at B=8192


def test_a_forced_plan_takes_any_shape_that_fits_and_refuses_the_rest(plan):
    assert plan(2048, 2048, 512, 2, force=1) is not None
    assert plan(64, 64, 40, 1, force=1) is None   # K not a multiple of 16
    assert plan(64, 66, 64, 1, force=1) is None   # N not a multiple of 4


def test_products_past_the_buffer_offset_range_do_not_take_the_narrow_body(plan):
    # The narrow body's buffer loads take 31-bit byte offsets from a block's
    # origin (up to 64 rows of A, K + 16 rows of B): a B of 2 GiB or more
    # goes to another body.
    assert plan(16, 16384, 32768, 8) is None          # (32768 + 16) x 16384 x 4 B >= 2^31
    assert plan(16, 16384, 32736, 8) is not None      # (32736 + 16) x 16384 x 4 B < 2^31
    assert plan(16, 64, 8 << 20, 8) is None           # 64 rows x 8 Mi k x 4 B = 2^31
