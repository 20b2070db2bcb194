#pragma once

// Compile-time autotuning of the FP32 matmul's K split (option `autotune`):
// the split count an Auto matmul uses is chosen by timing the candidates on
// the device, in place of the split rule's fixed thresholds
// (src/cuda/matmul_kernels.cu:352-367 in the reference, calibrated there on
// one GPU). Decisions are kept per (device, shape) for the process and, when
// MINICOMPILER_HIP_CACHE_DIR is set, in a text file there, so later processes
// reuse them without timing.

#include "minicompiler/hip/hip_backend.hpp"
#include "minicompiler/result.hpp"

#include <string>
#include <vector>

namespace minicompiler::hip {

// The candidate split counts for m x n x k on `cu_count` CUs: 1 (no split)
// and every power of two up to 64 that keeps at least 64 of K per split,
// gives at most four 128x128 tile-splits per CU and a workspace of at most
// 512 MiB; none above 1 once the unsplit tiles already give two per CU.
// The split rule's own choice is always among them.
std::vector<int> autotune_candidates(int m, int n, int k, int cu_count);

// The fastest candidate for an FP32 matmul m x n x k on the current device
// (`device` names it in the cache key), timed with the ahead-of-time kernels
// (double_buffered unsplit, split_k split) on scratch operands. Results of
// different split counts differ in rounding only (the partial sums are added
// in a fixed order), within the FP32 GEMM bound.
Result<int> autotune_fp32_splits(const DeviceInfo& device, int m, int n, int k);

// Decisions held by this process (for tests and reports).
std::size_t autotune_cached_decisions();

}  // namespace minicompiler::hip
