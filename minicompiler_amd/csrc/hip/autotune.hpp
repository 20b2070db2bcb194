#pragma once

// Compile-time autotuning of the FP32 matmul (option `autotune`): the K split
// and the tile configuration an Auto matmul uses are chosen by timing the
// candidates on the device, in place of the split rule's fixed thresholds
// (src/cuda/matmul_kernels.cu:352-367 in the reference, calibrated there on
// one GPU) and the ring planner's cost model. Decisions are kept per
// (device, shape) for the process and, when MINICOMPILER_HIP_CACHE_DIR is
// set, in a text file there, so later processes reuse them without timing.

#include "minicompiler/hip/hip_backend.hpp"
#include "minicompiler/result.hpp"

#include <string>
#include <vector>

namespace minicompiler::hip {

// An FP32 matmul's launch: `splits` K splits (1: double_buffered, more:
// split_k) on the ring configuration `ring_cfg` (MCHIP_RING_* of matmul.h;
// MCHIP_RING_NONE = 0: the planner's own choice).
struct Fp32Choice {
    int splits = 1;
    int ring_cfg = 0;
    bool operator==(const Fp32Choice& o) const { return splits == o.splits && ring_cfg == o.ring_cfg; }
};

// The candidates for m x n x k on `cu_count` CUs, the default first: the
// split rule's count on the planner's configuration. Products that already
// give two 128x128 tiles per CU, or that the ring cannot run (K not a
// multiple of 32, N not of 4), have no other. Otherwise, for each of the
// wide (128x128), mid (64x128) and thin (32x128) configurations: no split,
// and every power of two up to 64 that keeps at least 64 of K per split,
// gives at most four of that configuration's tile-splits per CU and a
// workspace of at most 512 MiB.
std::vector<Fp32Choice> autotune_candidates(int m, int n, int k, int cu_count);

// The fastest candidate for an FP32 matmul m x n x k on the current device
// (`device` names it in the cache key), timed with the ahead-of-time kernels
// on scratch operands; another candidate replaces the default only when more
// than 2% faster. `fold`: split candidates add their partials in the GEMM
// launch (mchip_launch_matmul_fold), as an executable with split_fold runs
// them; those decisions are kept apart (tag suffix "_fold"). Results of
// different split counts differ in rounding only (the partial sums are added
// in a fixed order), within the FP32 GEMM bound; the configuration does not
// change the bits.
Result<Fp32Choice> autotune_fp32(const DeviceInfo& device, int m, int n, int k, bool fold = false);

// Decisions held by this process (for tests and reports).
std::size_t autotune_cached_decisions();

}  // namespace minicompiler::hip
