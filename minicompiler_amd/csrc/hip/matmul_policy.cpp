#include "matmul_policy.hpp"

#include "matmul.h"

#include <algorithm>
#include <cstdint>

namespace minicompiler::hip {

int split_k_splits(int m, int n, int k, int cu_count, int blocks_per_cu) {
    const std::int64_t tiles = ((static_cast<std::int64_t>(m) + kSplitTileM - 1) / kSplitTileM) *
                               ((static_cast<std::int64_t>(n) + kSplitTileN - 1) / kSplitTileN);
    const std::int64_t cus = cu_count;
    // Nearly full: extra blocks gain less than the partials cost to write and sum.
    if (5 * tiles >= 4 * cus) return 1;
    // Up to half the CUs: one block per CU (a second block on some CUs only
    // makes a tail). Beyond that, up to two where a CU holds two.
    std::int64_t splits = (2 * tiles <= cus || blocks_per_cu < 2) ? cus / tiles : 2 * cus / tiles;
    splits = std::min<std::int64_t>(splits, k / 64);
    return static_cast<int>(std::max<std::int64_t>(splits, 1));
}

bool uses_split_k(MatmulKernel kernel) {
    switch (kernel) {
        case MatmulKernel::SplitK:
        case MatmulKernel::TensorCoreTf32:
        case MatmulKernel::TensorCoreBf16:
        case MatmulKernel::TensorCoreF16: return true;
        default: return false;
    }
}

int matmul_splits(MatmulKernel kernel, int m, int n, int k, int cu_count) {
    if (kernel == MatmulKernel::SplitK) return split_k_splits(m, n, k, cu_count);
    if (uses_split_k(kernel)) {
        return split_k_splits(m, n, k, cu_count, mchip_matmul_blocks_per_cu(static_cast<int>(kernel)));
    }
    return 1;
}

std::size_t matmul_workspace_bytes(MatmulKernel kernel, int m, int n, int splits) {
    if (!uses_split_k(kernel) || splits <= 1) return 0;
    return static_cast<std::size_t>(splits) * static_cast<std::size_t>(m) * static_cast<std::size_t>(n) * sizeof(float);
}

const char* matmul_kernel_name(MatmulKernel kernel) {
    switch (kernel) {
        case MatmulKernel::Auto: return "auto";
        case MatmulKernel::Naive: return "naive";
        case MatmulKernel::Tiled: return "tiled";
        case MatmulKernel::RegisterTiled128: return "register_tiled_128";
        case MatmulKernel::RegisterTiled64: return "register_tiled_64";
        case MatmulKernel::Vectorized: return "vectorized";
        case MatmulKernel::DoubleBuffered: return "double_buffered";
        case MatmulKernel::SplitK: return "split_k";
        case MatmulKernel::TensorCoreTf32: return "tensor_core_tf32";
        case MatmulKernel::TensorCoreBf16: return "tensor_core_bf16";
        case MatmulKernel::TensorCoreF16: return "tensor_core_f16";
    }
    return "?";
}

Result<MatmulKernel> matmul_kernel_from_name(const std::string& name) {
    for (int i = 0; i <= static_cast<int>(MatmulKernel::TensorCoreF16); ++i) {
        const auto k = static_cast<MatmulKernel>(i);
        if (name == matmul_kernel_name(k)) return k;
    }
    return Error{"unknown matmul kernel '" + name +
                 "' (auto, naive, tiled, register_tiled_128, register_tiled_64, vectorized, double_buffered, "
                 "split_k, tensor_core_tf32, tensor_core_bf16, tensor_core_f16)"};
}

MatmulKernel resolve_matmul_kernel(MatmulKernel kernel, int m, int n, int k, int cu_count) {
    if (kernel != MatmulKernel::Auto) return kernel;
    return split_k_splits(m, n, k, cu_count) > 1 ? MatmulKernel::SplitK : MatmulKernel::DoubleBuffered;
}

}  // namespace minicompiler::hip
