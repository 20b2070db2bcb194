// CPU oracle GEMM: row-major C[m,n] = A[m,k] B[k,n] in fp32 (the reference's
// Eigen `C.noalias() = A * B`, src/cpu/kernels.cpp:192-197). TEST
// INFRASTRUCTURE ONLY (see oracle.h). Cache-blocked over columns and K, four
// rows of C per pass so each loaded row segment of B feeds four rows; fp32
// accumulation along K with fused multiply-adds (as Eigen's AVX2+FMA kernel
// accumulates). Rows are split over orc_set_threads() threads.

#include "oracle.h"

#include <algorithm>
#include <cstring>
#include <thread>
#include <vector>

namespace {

constexpr int64_t kColBlock = 512;
constexpr int64_t kDepthBlock = 128;

void gemm_rows(const float* a, const float* b, float* c, int64_t r0, int64_t r1, int64_t k, int64_t n) {
    for (int64_t r = r0; r < r1; ++r) std::memset(c + r * n, 0, static_cast<size_t>(n) * sizeof(float));
    for (int64_t j0 = 0; j0 < n; j0 += kColBlock) {
        const int64_t j1 = std::min(n, j0 + kColBlock);
        for (int64_t t0 = 0; t0 < k; t0 += kDepthBlock) {
            const int64_t t1 = std::min(k, t0 + kDepthBlock);
            int64_t r = r0;
            for (; r + 4 <= r1; r += 4) {
                float* c0 = c + r * n;
                float* c1 = c0 + n;
                float* c2 = c1 + n;
                float* c3 = c2 + n;
                for (int64_t t = t0; t < t1; ++t) {
                    const float a0 = a[r * k + t], a1 = a[(r + 1) * k + t], a2 = a[(r + 2) * k + t],
                                a3 = a[(r + 3) * k + t];
                    const float* bt = b + t * n;
                    for (int64_t j = j0; j < j1; ++j) {
                        const float bv = bt[j];
                        c0[j] += a0 * bv;
                        c1[j] += a1 * bv;
                        c2[j] += a2 * bv;
                        c3[j] += a3 * bv;
                    }
                }
            }
            for (; r < r1; ++r) {
                float* cr = c + r * n;
                for (int64_t t = t0; t < t1; ++t) {
                    const float av = a[r * k + t];
                    const float* bt = b + t * n;
                    for (int64_t j = j0; j < j1; ++j) cr[j] += av * bt[j];
                }
            }
        }
    }
}

}  // namespace

extern "C" int orc_matmul(const float* a, const float* b, float* c, int64_t m, int64_t k, int64_t n) {
    if (m < 1 || n < 1 || k < 1) return 1;
    const int64_t threads = std::max<int64_t>(1, std::min<int64_t>(orc_get_threads(), (m + 3) / 4));
    if (threads == 1) {
        gemm_rows(a, b, c, 0, m, k, n);
        return 0;
    }
    std::vector<std::thread> pool;
    for (int64_t w = 0; w < threads; ++w) {
        // Row ranges in multiples of 4 so the register blocking stays whole.
        const int64_t quads = (m + 3) / 4;
        const int64_t b0 = std::min(m, quads * w / threads * 4), b1 = std::min(m, quads * (w + 1) / threads * 4);
        if (b0 < b1) pool.emplace_back(gemm_rows, a, b, c, b0, b1, k, n);
    }
    for (auto& t : pool) t.join();
    return 0;
}
