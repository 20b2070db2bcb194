/* Launchers of the AOT-compiled gfx950 matmul kernels (matmul_fp32.hip,
 * matmul_mfma16.hip). Plain C ABI: the host C++ calls them without HIP
 * headers. `kernel` takes the values of minicompiler::hip::MatmulKernel.
 * Each returns 0 or a hipError_t value: hipErrorInvalidValue (1) for an
 * unresolved Auto, a bad shape or a missing workspace, hipErrorNotSupported
 * (801) for a kernel gfx950 cannot run (TensorCoreTf32).
 *
 * Replaces the reference's launch_matmul / launch_tensor_core /
 * sum_split_partials (src/cuda/matmul_kernels.hpp:36-59). */
#pragma once

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { MCHIP_DTYPE_F32 = 0, MCHIP_DTYPE_BF16 = 1, MCHIP_DTYPE_F16 = 2 };

/* C[m,n] = A[m,k] B[k,n], row-major fp32. A kernel that splits K reads
 * `splits` and, above 1, `workspace` (splits * m * n floats). */
int mchip_launch_matmul(int kernel, const float* a, const float* b, float* c, int m, int n, int k, void* stream,
                        int splits, float* workspace);

/* The matrix-core kernels on inputs already in bf16 or fp16 in device memory
 * (dtype MCHIP_DTYPE_BF16 / MCHIP_DTYPE_F16), fp32 accumulation and output. */
int mchip_launch_matmul_lowp(int kernel, int dtype, const void* a, const void* b, float* c, int m, int n, int k,
                             void* stream, int splits, float* workspace);

/* Packed A for the bf16/fp16 256x256-tile kernel (gemm_mfma16_fast.h): the
 * elements it holds for an m x k operand (m rounded up to 256 rows), 16-bit
 * row-major A packed, fp32 A rounded and packed in one pass (k a multiple
 * of 64, pointers 16-byte aligned), and the product on packed A (the shapes
 * and alignment of the fast kernel; same bits as on row-major A). */
long long mchip_packed_a16_elements(int m, int k);
int mchip_pack_a16(const void* a, void* packed, int m, int k, void* stream);
int mchip_convert_pack_a_f32(int dtype, const float* a, void* packed, int m, int k, void* stream);
int mchip_launch_matmul_lowp_packed(int kernel, int dtype, const void* a_packed, const void* b, float* c, int m, int n,
                                    int k, void* stream);

/* C = sum over z of partial[z * count + i], added in z order. */
int mchip_sum_split_partials(const float* partial, float* c, size_t count, int splits, void* stream);

/* Blocks of the bf16/fp16 256x256-tile kernel (gemm_mfma16_fast.h) for an
 * m x n product on `cu_count` CUs: one per tile, plus one more for each of
 * the last tiles when they would fill at most half of the CUs in their round
 * (those tiles then run as two 128-row halves). */
unsigned mchip_mfma16_fast_grid(int m, int n, int cu_count);

/* Whether the bf16/fp16 256x256-tile kernel takes an m x n x k product: K a
 * multiple of 64, N a multiple of 8 (at least 8), and every byte offset its
 * buffer loads take from a tile's origin below 2^31 (256 rows of A, K + 32
 * rows of B). Alignment is the caller's to check. */
int mchip_mfma16_fast_fits(int m, int n, int k);

/* Whether gfx950 runs `kernel` (all but TensorCoreTf32). */
int mchip_matmul_supported(int kernel);

/* Resident blocks per CU of the kernel that runs `kernel` (occupancy), or 1. */
int mchip_matmul_blocks_per_cu(int kernel);

/* How the FP32 matrix-core ring body (double_buffered and split_k) runs an
 * m x n x k product in `depth` K splits on `cu_count` CUs, ignoring operand
 * alignment (16-byte aligned A, B and C are required too):
 *   MCHIP_RING_NONE  the shape does not fit it (K not a multiple of 32, or N
 *                    not a multiple of 4): the two-stage body runs instead;
 *   MCHIP_RING_BIG   one persistent block of 4 waves per CU, 256x256 tiles;
 *   MCHIP_RING_WIDE  up to two persistent blocks of 4 waves per CU, 128x128
 *                    tiles, the fetch staged through registers;
 *   MCHIP_RING_THIN  for m <= 32: 32x128 tiles, 6 LDS stages;
 *   MCHIP_RING_WIDE8 128x128 tiles in one block of 8 waves per CU, in place
 *                    of wide when the product has at most one tile (or
 *                    tile-split) per CU.
 * The choice minimises (rounds of tiles per CU) x (work per tile) / (the
 * configuration's measured efficiency). *grid receives the number of
 * blocks, *block the lanes per block.
 *   MCHIP_RING_MID   64x128 tiles, up to two blocks per CU: never chosen
 *                    here, only when forced (the autotuner times it).
 * mchip_f32_ring_plan_cfg with cfg != MCHIP_RING_NONE forces that
 * configuration (thin then at any m), if the shape fits the ring at all. */
enum {
    MCHIP_RING_NONE = 0,
    MCHIP_RING_WIDE = 1,
    MCHIP_RING_MID = 2,
    MCHIP_RING_BIG = 3,
    MCHIP_RING_THIN = 4,
    MCHIP_RING_NARROW = 5,
    MCHIP_RING_WIDE8 = 6
};
int mchip_f32_ring_plan(int m, int n, int k, int depth, int cu_count, unsigned* grid, unsigned* block);
int mchip_f32_ring_plan_cfg(int m, int n, int k, int depth, int cu_count, int cfg, unsigned* grid, unsigned* block);


/* The narrow-tile body (gemm_f32_narrow.h) in its tile shapes. */
enum {
    MCHIP_NARROW_32X64 = 0,         /* 32x64 tiles */
    MCHIP_NARROW_16X64_STREAM = 1,  /* 16x64 tiles, B streamed: m <= 16 */
    MCHIP_NARROW_16X64 = 2,         /* 16x64 tiles */
    MCHIP_NARROW_16X32 = 3,         /* 16x32 tiles */
    MCHIP_NARROW_64X64 = 4,         /* 64x64 tiles */
};
int mchip_narrow_rows(int shape);
int mchip_narrow_cols(int shape);

/* The narrow-tile body, which the split_k rung runs for products whose
 * tiles number at most one per CU (two for 64x64 tiles). With K <= 2048, a
 * tile shape that gives more than half the CUs a tile runs unsplit (the
 * first of 64x64, 32x64, 16x64, 16x32 that does); otherwise 32x64 tiles (16x64, B streamed, for m <= 16)
 * with K cut into *splits ranges of *k_split (a multiple of 16), at most
 * max_splits of them, so that tiles x ranges stays within the CUs. Its
 * accumulation order is its own (16x16x4 MFMAs, K pieces per wave added
 * in wave order, then the ranges in range order), not the ring body's.
 * Returns 1 and fills *shape (MCHIP_NARROW_*), *splits and *k_split when
 * the plan runs the product on it (force: whenever the shape fits: k a
 * multiple of 16, n of 4), else 0. */
int mchip_f32_narrow_plan(int m, int n, int k, int max_splits, int cu_count, int force, int* shape, int* splits,
                          int* k_split);

/* The narrow-tile body directly: `rows` 16 (m <= 16) or 32, K in `splits`
 * ranges; above one range the partials go to `workspace` (splits * m * n
 * floats) and are summed in range order. */
int mchip_launch_narrow(const float* a, const float* b, float* c, int m, int n, int k, void* stream, int splits,
                        int rows, float* workspace);

/* mchip_launch_matmul with the ring configuration forced (MCHIP_RING_NONE:
 * the plan's own) for double_buffered and split_k (MCHIP_RING_NARROW: the
 * narrow-tile body, split_k only); hipErrorInvalidValue
 * when that configuration cannot run the product (K not a multiple of 32, N
 * not of 4, operands not 16-byte aligned) or for other kernels. */
int mchip_launch_matmul_cfg(int kernel, const float* a, const float* b, float* c, int m, int n, int k, void* stream,
                            int splits, float* workspace, int ring_cfg);

/* The number of K ranges mchip_launch_matmul_cfg runs for `kernel` when
 * given `splits` (16-byte aligned operands, a workspace): `splits` is an
 * upper bound, since the narrow-tile body of split_k runs fewer ranges when
 * its plan fills the CUs with fewer (256x256x16384 with 64 splits runs 8);
 * 1 for kernels that do not split; 0 for invalid sizes or a configuration
 * that cannot run the product. */
int mchip_matmul_k_ranges(int kernel, int m, int n, int k, int splits, int ring_cfg);
int mchip_tensor_core_k_ranges(int k, int splits);

/* mchip_launch_matmul_cfg for split_k that adds the K splits' partials in
 * the GEMM launch itself where the ring or narrow body runs the product: the
 * last block to finish a split of a C tile adds the tile's partials in split
 * order (the bits of the separate sum) and stores C; no sum launch.
 * `counters`: mchip_split_counter_bytes(m, n) bytes of device memory, zero
 * before the first launch and left zero by every launch; launches that share
 * them must not overlap. Other kernels, or counters null: as
 * mchip_launch_matmul_cfg. */
unsigned long long mchip_split_counter_bytes(int m, int n);
/* 1 when mchip_launch_matmul_fold with counters adds the partials of this
 * split_k product (16-byte aligned operands and workspace) in the GEMM
 * launch: the plan runs it on the ring or narrow body in several K splits. */
int mchip_split_k_folds(int m, int n, int k, int splits, int ring_cfg);
int mchip_launch_matmul_fold(int kernel, const float* a, const float* b, float* c, int m, int n, int k, void* stream,
                             int splits, float* workspace, int ring_cfg, unsigned* counters);

/* mchip_launch_matmul with the split-K partials in the library's per-device
 * scratch array (matmul_noalloc.hip) instead of a caller workspace; no
 * device memory is allocated. hipErrorInvalidValue when the partials
 * (mchip_noalloc_required_bytes) exceed mchip_noalloc_scratch_bytes().
 * Calls that overlap on one GPU race on the array. */
int mchip_launch_matmul_noalloc(int kernel, const float* a, const float* b, float* c, int m, int n, int k,
                                void* stream, int splits);
unsigned long long mchip_noalloc_scratch_bytes(void);
unsigned long long mchip_noalloc_required_bytes(int kernel, int m, int n, int splits);

/* Elementwise fp32 -> bf16/fp16 (round to nearest even), for staging. */
int mchip_convert_f32(int dtype, const float* in, void* out, size_t count, void* stream);

#ifdef __cplusplus
}
#endif
