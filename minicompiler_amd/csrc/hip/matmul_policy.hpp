#pragma once

// Host-side matmul policy: the split-K rule, workspace sizing and kernel
// names (reference: src/cuda/matmul_kernels.hpp:12-34, matmul_kernels.cu:352-383).

#include "minicompiler/hip/hip_backend.hpp"

#include <cstddef>

namespace minicompiler::hip {

// Output tile every split-K-capable kernel uses.
inline constexpr int kSplitTileM = 128;
inline constexpr int kSplitTileN = 128;

// Ways to divide K for m x n x k on `cu_count` CUs, from the number of
// 128x128 output tiles and the blocks of the kernel a CU holds at once:
// none when the tiles cover at least 80% of the CUs; one block per CU when
// they cover at most half, or whenever a CU holds a single block; up to two
// blocks per CU in between; and never below 64 of K per split.
int split_k_splits(int m, int n, int k, int cu_count, int blocks_per_cu = 2);

// SplitK and the TensorCore* kernels divide K.
bool uses_split_k(MatmulKernel kernel);

int matmul_splits(MatmulKernel kernel, int m, int n, int k, int cu_count);

// splits * m * n floats for a kernel that splits K into more than one piece.
std::size_t matmul_workspace_bytes(MatmulKernel kernel, int m, int n, int splits);

// The K each split covers (whole multiples of `step`) and the resulting depth.
inline int split_size(int k, int splits, int step) {
    if (splits <= 1) return k > 1 ? k : 1;
    const int per = (k + splits - 1) / splits;
    return (per + step - 1) / step * step;
}
inline int split_depth(int k, int k_split) {
    const int d = (k + k_split - 1) / k_split;
    return d > 1 ? d : 1;
}

}  // namespace minicompiler::hip
