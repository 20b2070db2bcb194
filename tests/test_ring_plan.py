"""The FP32 ring planner (mchip_f32_ring_plan_cfg, host logic, no GPU): the
tile configuration, grid and block it gives the bench's and the MLP's
products on 256 CUs, and what a forced configuration gives. Configurations:
1 wide (128x128, 4 waves), 2 mid, 3 big (256x256), 4 thin (32x128),
6 wide8 (128x128, 8 waves)."""

import ctypes

import pytest

NONE, WIDE, MID, BIG, THIN, WIDE8 = 0, 1, 2, 3, 4, 6


@pytest.fixture(scope="module")
def plan(mc):
    f = mc.library().mchip_f32_ring_plan_cfg
    f.argtypes = [ctypes.c_int] * 6 + [ctypes.POINTER(ctypes.c_uint)] * 2
    f.restype = ctypes.c_int

    def run(m, n, k, depth=1, cfg=NONE, cus=256):
        grid, block = ctypes.c_uint(), ctypes.c_uint()
        got = f(m, n, k, depth, cus, cfg, ctypes.byref(grid), ctypes.byref(block))
        return got, grid.value, block.value

    return run


@pytest.mark.parametrize("m,n,k,depth,want", [
    (8192, 8192, 8192, 1, (WIDE, 512, 256)),     # 4096 tiles of 128x128, two persistent blocks per CU
    (4096, 4096, 4096, 1, (WIDE, 512, 256)),
    (8192, 2048, 512, 1, (WIDE, 512, 256)),      # the MLP's GEMM1 at B=8192
    (8192, 512, 2048, 1, (WIDE8, 256, 512)),     # its GEMM2: one 128x128 tile per CU
    (2048, 2048, 2048, 1, (WIDE8, 256, 512)),
    (1024, 1024, 1024, 4, (WIDE8, 256, 512)),    # 64 tiles x 4 splits
    (16, 4096, 4096, 8, (THIN, 256, 256)),       # M <= 32
])
def test_the_planner_for_the_bench_and_mlp_shapes(plan, m, n, k, depth, want):
    assert plan(m, n, k, depth) == want


def test_a_forced_configuration_keeps_its_tiles_in_persistent_blocks(plan):
    assert plan(8192, 512, 2048, cfg=WIDE) == (WIDE, 256, 256)      # 256 tiles, up to two blocks per CU
    assert plan(4096, 4096, 4096, cfg=WIDE) == (WIDE, 512, 256)     # 1024 tiles
    assert plan(8192, 512, 2048, cfg=BIG) == (BIG, 64, 256)         # 64 tiles of 256x256
    assert plan(1000, 1024, 512, cfg=MID) == (MID, 128, 256)        # 16 x 8 tiles of 64x128
    assert plan(1000, 1024, 512, cfg=WIDE8) == (WIDE8, 64, 512)


def test_shapes_the_ring_cannot_take(plan):
    assert plan(64, 64, 40)[0] == NONE   # K not a multiple of 32
    assert plan(64, 66, 64)[0] == NONE   # N not a multiple of 4


def test_products_past_the_buffer_offset_range_do_not_take_the_ring(plan):
    # The ring's buffer loads and stores take 31-bit byte offsets from a
    # tile's origin (256 rows of A, K + 32 rows of B, 256 rows of C).
    assert plan(64, 16384, 32768)[0] == NONE          # (32768 + 32) x 16384 x 4 B >= 2^31
    assert plan(64, 16384, 32704)[0] != NONE          # (32704 + 32) x 16384 x 4 B < 2^31
    assert plan(64, 64, 2 << 20)[0] == NONE           # 256 rows x 2 Mi k x 4 B = 2^31
    assert plan(64, 2 << 20, 32)[0] == NONE           # 256 rows of C x 2 Mi n x 4 B = 2^31
    assert plan(64, (2 << 20) - 4, 32)[0] != NONE     # one column chunk fewer


def test_the_bf16_fast_kernel_bounds_its_offsets(mc):
    f = mc.library().mchip_mfma16_fast_fits
    f.argtypes = [ctypes.c_int] * 3
    f.restype = ctypes.c_int
    assert f(8192, 8192, 8192) == 1
    assert f(4096, 14336, 4096) == 1
    assert f(64, 8, 64) == 1
    assert f(64, 8, 96) == 0                          # K not a multiple of 64
    assert f(64, 12, 64) == 0                         # N not a multiple of 8
    assert f(64, 32768, 32768) == 0                   # 2 x (32768 + 32) x 32768 B >= 2^31
    assert f(64, 32768, 32704) == 1                   # 2 x (32704 + 32) x 32768 B < 2^31
    assert f(64, 64, 4 << 20) == 0                    # 2 x 256 rows x 4 Mi k B = 2^31
