// FP32 matmul kernels for gfx950 (CDNA4), ahead-of-time compiled. They take
// the place of the reference's FP32 ladder (src/cuda/matmul_kernels.cu:18-417).
// C[m,n] = A[m,k] B[k,n], row-major fp32, any shape.
//
// The ladder, one step of optimisation each:
//   naive              one output per lane, operands from global memory
//   tiled              32x32 LDS tiles, one output per lane
//   register_tiled_*   128x128 / 64x64 LDS tiles, 8x8 / 4x4 outputs per lane
//   vectorized         128x128x32 tiles, 16-byte global loads, the products on
//                      the FP32 matrix cores (v_mfma_f32_32x32x2_f32)
//   double_buffered    vectorized with two LDS stages: the next tile's global
//                      loads are in flight during the current tile's MFMAs
//   split_k            double_buffered with K split over the grid's depth and
//                      a fixed-order (deterministic) sum of the partials
//
// double_buffered and split_k run the ring body (gemm_f32_ring.h) where the
// shape allows: direct global -> LDS loads, persistent blocks walking their
// tiles (and K splits) with an XCD-aware order, in one of three
// configurations (256x256 tiles; 128x128 tiles with two blocks per CU;
// 128x128 tiles with four stages; 32x128 tiles for M <= 32). Its arithmetic
// is the two-stage body's, bit for bit.

#include "matmul.h"

#include <hip/hip_runtime.h>

#include "gemm_f32_mfma.h"
#include "gemm_split_arrival.h"
#include "gemm_f32_ring.h"
#include "gemm_f32_narrow.h"

#include <algorithm>
#include <atomic>
#include <cstddef>
#include <cstdint>

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// MatmulKernel values (minicompiler/hip/hip_backend.hpp).
enum Kernel {
    kAuto = 0,
    kNaive,
    kTiled,
    kRegisterTiled128,
    kRegisterTiled64,
    kVectorized,
    kDoubleBuffered,
    kSplitK,
    kTensorCoreTf32,
    kTensorCoreBf16,
    kTensorCoreF16,
};

// ---------------------------------------------------------------- naive

__global__ void __launch_bounds__(256) matmul_naive(const float* __restrict__ a, const float* __restrict__ b,
                                                    float* __restrict__ c, int m, int n, int k) {
    const int col = blockIdx.x * 16 + threadIdx.x;
    const int row = blockIdx.y * 16 + threadIdx.y;
    if (row >= m || col >= n) return;
    float acc = 0.0f;
    const float* ar = a + static_cast<std::ptrdiff_t>(row) * k;
    for (int t = 0; t < k; ++t) acc += ar[t] * b[static_cast<std::ptrdiff_t>(t) * n + col];
    c[static_cast<std::ptrdiff_t>(row) * n + col] = acc;
}

// ---------------------------------------------------------------- tiled

constexpr int kTile = 32;

__global__ void __launch_bounds__(1024) matmul_tiled(const float* __restrict__ a, const float* __restrict__ b,
                                                     float* __restrict__ c, int m, int n, int k) {
    __shared__ float at[kTile][kTile + 1];
    __shared__ float bt[kTile][kTile + 1];
    const int tx = threadIdx.x, ty = threadIdx.y;
    const int row = blockIdx.y * kTile + ty, col = blockIdx.x * kTile + tx;
    float acc = 0.0f;
    for (int k0 = 0; k0 < k; k0 += kTile) {
        at[ty][tx] = (row < m && k0 + tx < k) ? a[static_cast<std::ptrdiff_t>(row) * k + k0 + tx] : 0.0f;
        bt[ty][tx] = (k0 + ty < k && col < n) ? b[static_cast<std::ptrdiff_t>(k0 + ty) * n + col] : 0.0f;
        __syncthreads();
#pragma unroll
        for (int t = 0; t < kTile; ++t) acc += at[ty][t] * bt[t][tx];
        __syncthreads();
    }
    if (row < m && col < n) c[static_cast<std::ptrdiff_t>(row) * n + col] = acc;
}

// ---------------------------------------------------------------- register tiled
//
// 256 lanes as an R x C grid (R = BM/TM, C = BN/TN). Lane (r, c) owns rows
// r + R*i and columns c + C*j of the block tile: along a wave the B reads are
// consecutive words and the A reads broadcasts. A is staged transposed (k
// major) so both operands are read along a row of LDS.

template <int BM, int BN, int BK, int TM, int TN>
__global__ void __launch_bounds__(256) matmul_register_tiled(const float* __restrict__ a, const float* __restrict__ b,
                                                             float* __restrict__ c, int m, int n, int k) {
    constexpr int R = BM / TM, C = BN / TN;
    static_assert(R * C == 256, "256 lanes");
    __shared__ float as[BK][BM];
    __shared__ float bs[BK][BN];
    const int tid = threadIdx.x;
    const int lr = tid / C, lc = tid % C;
    const int row0 = blockIdx.y * BM, col0 = blockIdx.x * BN;
    float acc[TM][TN] = {};
    for (int k0 = 0; k0 < k; k0 += BK) {
        for (int e = tid; e < BM * BK; e += 256) {
            const int r = e / BK, kk = e % BK;
            const int gr = row0 + r, gk = k0 + kk;
            as[kk][r] = (gr < m && gk < k) ? a[static_cast<std::ptrdiff_t>(gr) * k + gk] : 0.0f;
        }
        for (int e = tid; e < BK * BN; e += 256) {
            const int kk = e / BN, cc = e % BN;
            const int gk = k0 + kk, gc = col0 + cc;
            bs[kk][cc] = (gk < k && gc < n) ? b[static_cast<std::ptrdiff_t>(gk) * n + gc] : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int t = 0; t < BK; ++t) {
            float av[TM], bv[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) av[i] = as[t][lr + R * i];
#pragma unroll
            for (int j = 0; j < TN; ++j) bv[j] = bs[t][lc + C * j];
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) acc[i][j] += av[i] * bv[j];
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const int gr = row0 + lr + R * i;
        if (gr >= m) continue;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int gc = col0 + lc + C * j;
            if (gc < n) c[static_cast<std::ptrdiff_t>(gr) * n + gc] = acc[i][j];
        }
    }
}

// ---------------------------------------------------------------- FP32 MFMA
//
// The body lives in gemm_f32_mfma.h (also compiled at run time with fused
// epilogues); here it is instantiated with the identity epilogue.

template <bool kDouble, bool kVec>
__global__ void __launch_bounds__(256, 2) matmul_mfma_f32(const float* __restrict__ a, const float* __restrict__ b,
                                                          float* __restrict__ c, int m, int n, int k, int k_split,
                                                          float* __restrict__ partial) {
    mc_gemm_f32_mfma<kDouble, kVec>(a, b, c, m, n, k, k_split, partial, McGemmStore{});
}

using RingBig = McRingBig;
using RingWide = McRingWide;
using RingWide8 = McRingWide8;
using RingThin = McRingThin;
using RingMid = McRingMid;
constexpr int kRBKRing = RingWide::kBK;

template <class Cfg, int kBlocksPerCu>
__global__ void __launch_bounds__(Cfg::kThreads, kBlocksPerCu)
    matmul_ring_f32(const float* __restrict__ a, const float* __restrict__ b, float* __restrict__ c, int m, int n,
                    int k, int k_split, int depth, float* __restrict__ partial, unsigned* __restrict__ counters) {
    mc_gemm_f32_ring<Cfg>(a, b, c, m, n, k, k_split, depth, partial, counters, McGemmStore{});
}

// ---------------------------------------------------------------- narrow tiles

struct McIdentity {
    __device__ __forceinline__ float operator()(float v, unsigned) const { return v; }
};

template <class Cfg>
__global__ void __launch_bounds__(Cfg::kThreads) matmul_narrow_f32(const float* __restrict__ a,
                                                                    const float* __restrict__ b, float* __restrict__ c,
                                                                    int m, int n, int k, int k_split, int depth,
                                                                    float* __restrict__ partial,
                                                                    unsigned* __restrict__ counters) {
    mc_gemm_f32_narrow<Cfg>(a, b, c, m, n, k, k_split, depth, partial, counters, McIdentity{});
}

// ---------------------------------------------------------------- split-K sum

// c[i] = partial[0][i] + partial[1][i] + ... in split order (a left fold,
// starting from split 0's value so a -0.0 stays -0.0). T is float or f32x4.
// The partials are read once, with non-temporal loads: left in the L2s,
// their lines slowed the next launch's GEMM writing the same workspace
// (1024^3 in 4 splits, graph-timed on an MI355X with one workspace for all
// launches: 31.1 us with plain loads, 29.0 with non-temporal ones; 27.2
// against 26.8 us with a workspace per launch).
// A lane loads kChunk splits before it adds any: split indices past the last
// are clamped to it (an in-bounds reload) and their adds skipped, so all
// kChunk loads are independent and in flight together. A lane that walked
// the splits one load at a time waited a full memory latency per split: 64
// splits of a 256x256 product took 16.7 us for 16 MiB of partials.
template <typename T, int kChunk>
__global__ void __launch_bounds__(256) sum_splits_chunked(const T* __restrict__ partial, T* __restrict__ c,
                                                          std::size_t count, int splits) {
    const std::size_t stride = static_cast<std::size_t>(gridDim.x) * 256;
    for (std::size_t i = static_cast<std::size_t>(blockIdx.x) * 256 + threadIdx.x; i < count; i += stride) {
        T s = __builtin_nontemporal_load(partial + i);
        for (int z0 = 1; z0 < splits; z0 += kChunk) {
            T p[kChunk];
#pragma unroll
            for (int j = 0; j < kChunk; ++j) {
                const int z = z0 + j < splits ? z0 + j : splits - 1;
                p[j] = __builtin_nontemporal_load(partial + static_cast<std::size_t>(z) * count + i);
            }
#pragma unroll
            for (int j = 0; j < kChunk; ++j)
                if (z0 + j < splits) s += p[j];
        }
        c[i] = s;
    }
}

bool aligned16(const void* p) { return reinterpret_cast<std::uintptr_t>(p) % 16 == 0; }

int split_len(int k, int splits, int step) {
    if (splits <= 1) return std::max(k, 1);
    const int per = (k + splits - 1) / splits;
    return (per + step - 1) / step * step;
}

// CUs of the current device, asked once per device.
int device_cu_count() {
    static std::atomic<int> cache[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (dev >= 0 && dev < 64) {
        const int c = cache[dev].load(std::memory_order_relaxed);
        if (c > 0) return c;
    }
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    if (dev >= 0 && dev < 64) cache[dev].store(cus, std::memory_order_relaxed);
    return cus;
}

template <class Cfg>
void narrow_kernel(const float* a, const float* b, float* c, int m, int n, int k, hipStream_t s, int k_split,
                   int depth, float* part, unsigned* counters) {
    const dim3 grid(((n + Cfg::kCols - 1) / Cfg::kCols) * depth * ((m + Cfg::kRows - 1) / Cfg::kRows));
    hipLaunchKernelGGL((matmul_narrow_f32<Cfg>), grid, dim3(Cfg::kThreads), 0, s, a, b, c, m, n, k, k_split, depth,
                       part, counters);
}

// The narrow-tile body in tile shape `shape` on `depth` K ranges of
// k_split, the partials summed in range order when there are several: in
// the launch when `counters` (zeroed, one per tile) is given, else by a
// separate launch.
int launch_narrow(const float* a, const float* b, float* c, int m, int n, int k, hipStream_t s, int shape,
                  int k_split, int depth, float* workspace, unsigned* counters) {
    float* dst = depth > 1 ? workspace : c;
    if (!aligned16(a) || !aligned16(b) || dst == nullptr) return hipErrorInvalidValue;
    if (shape == MCHIP_NARROW_16X64_STREAM && m > 16) return hipErrorInvalidValue;
    float* part = depth > 1 ? workspace : nullptr;
    unsigned* ctr = depth > 1 ? counters : nullptr;
    switch (shape) {
        case MCHIP_NARROW_32X64: narrow_kernel<McNarrow32>(a, b, c, m, n, k, s, k_split, depth, part, ctr); break;
        case MCHIP_NARROW_16X64_STREAM: narrow_kernel<McNarrow16>(a, b, c, m, n, k, s, k_split, depth, part, ctr); break;
        case MCHIP_NARROW_16X64: narrow_kernel<McNarrow16x64>(a, b, c, m, n, k, s, k_split, depth, part, ctr); break;
        case MCHIP_NARROW_16X32: narrow_kernel<McNarrow16x32>(a, b, c, m, n, k, s, k_split, depth, part, ctr); break;
        case MCHIP_NARROW_64X64: narrow_kernel<McNarrow64>(a, b, c, m, n, k, s, k_split, depth, part, ctr); break;
        default: return hipErrorInvalidValue;
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess || depth == 1 || ctr != nullptr) return e;
    return mchip_sum_split_partials(workspace, c, static_cast<std::size_t>(m) * n, depth, s);
}

// How launch_mfma_f32 runs a product: the body (narrow tiles, a ring
// configuration, or the two-stage body), its K ranges and grid. `a16`...:
// whether A, B, C and the workspace are 16-byte aligned.
struct MfmaPlan {
    int status = hipSuccess;
    bool narrow = false;
    int shape = 0;  // MCHIP_NARROW_* when narrow
    int ring = MCHIP_RING_NONE;
    int k_split = 0, depth = 1;
    unsigned ring_grid = 0, ring_block = 0;
    bool vec = false;
    // The split's partials go to a workspace and a body that can add them
    // in its own launch (ring or narrow) runs it.
    bool can_fold() const { return status == hipSuccess && depth > 1 && (narrow || ring != MCHIP_RING_NONE); }
};

MfmaPlan plan_mfma_f32(bool double_buffer, bool a16, bool b16, bool c16, bool ws16, bool has_ws, int m, int n, int k,
                       int splits, int ring_cfg, bool split_k) {
    MfmaPlan p;
    // split_k on the narrow-tile body when the plan (or the caller) takes it,
    // with at most the caller's split count (its workspace's size).
    if (split_k && (ring_cfg == MCHIP_RING_NONE || ring_cfg == MCHIP_RING_NARROW) && a16 && b16) {
        int shape = 0, ns = 0, nk = 0;
        if (mchip_f32_narrow_plan(m, n, k, std::max(splits, 1), device_cu_count(), ring_cfg == MCHIP_RING_NARROW,
                                  &shape, &ns, &nk)) {
            p.narrow = true;
            p.shape = shape;
            p.k_split = nk;
            p.depth = ns;
            if (ns > 1 && !has_ws) p.status = hipErrorInvalidValue;  // as the ring would
            return p;
        }
    }
    if (ring_cfg == MCHIP_RING_NARROW) {
        p.status = hipErrorInvalidValue;
        return p;
    }
    p.k_split = split_len(k, splits, kMBK);
    p.depth = std::max(1, (k + p.k_split - 1) / p.k_split);
    if (p.depth > 1 && !has_ws) {
        p.status = hipErrorInvalidValue;
        return p;
    }
    p.vec = n % 4 == 0 && k % 4 == 0 && a16 && b16;
    // The ring body stores C (or a split's partial) 4, 8 or 16 bytes at a
    // time: the destination must be 16-byte aligned, as the reference
    // requires of the workspace (matmul_kernels.cu:324).
    const bool dest_aligned = p.depth > 1 ? ws16 : c16;
    p.ring = double_buffer && p.vec && dest_aligned
                 ? mchip_f32_ring_plan_cfg(m, n, k, p.depth, device_cu_count(), ring_cfg, &p.ring_grid, &p.ring_block)
                 : MCHIP_RING_NONE;
    if (ring_cfg != MCHIP_RING_NONE && p.ring != ring_cfg) p.status = hipErrorInvalidValue;
    return p;
}

// `counters` (zeroed, one per tile; may be null): where the ring or narrow
// body runs the split, the launch adds the partials itself.
int launch_mfma_f32(bool double_buffer, const float* a, const float* b, float* c, int m, int n, int k,
                    hipStream_t stream, int splits, float* workspace, int ring_cfg, bool split_k,
                    unsigned* counters = nullptr) {
    const MfmaPlan p = plan_mfma_f32(double_buffer, aligned16(a), aligned16(b), aligned16(c), aligned16(workspace),
                                     workspace != nullptr, m, n, k, splits, ring_cfg, split_k);
    if (p.status != hipSuccess) return p.status;
    if (p.narrow) return launch_narrow(a, b, c, m, n, k, stream, p.shape, p.k_split, p.depth, workspace, counters);
    const int k_split = p.k_split, depth = p.depth;
    const dim3 grid((n + kMBN - 1) / kMBN, (m + kMBM - 1) / kMBM, depth);
    const bool vec = p.vec;
    float* out_ws = depth > 1 ? workspace : nullptr;
    const unsigned ring_grid = p.ring_grid, ring_block = p.ring_block;
    const int ring = p.ring;
    // The ring's fold stores C 16 bytes at a time.
    unsigned* ctr = p.can_fold() && aligned16(c) ? counters : nullptr;
    if (ring == MCHIP_RING_THIN) {
        hipLaunchKernelGGL((matmul_ring_f32<RingThin, 1>), dim3(ring_grid), dim3(ring_block), 0, stream, a, b, c, m, n,
                           k, k_split, depth, out_ws, ctr);
    } else if (ring == MCHIP_RING_BIG) {
        hipLaunchKernelGGL((matmul_ring_f32<RingBig, 1>), dim3(ring_grid), dim3(ring_block), 0, stream, a, b, c, m, n,
                           k, k_split, depth, out_ws, ctr);
    } else if (ring == MCHIP_RING_WIDE8) {
        hipLaunchKernelGGL((matmul_ring_f32<RingWide8, 1>), dim3(ring_grid), dim3(ring_block), 0, stream, a, b, c, m, n,
                           k, k_split, depth, out_ws, ctr);
    } else if (ring == MCHIP_RING_WIDE) {
        hipLaunchKernelGGL((matmul_ring_f32<RingWide, 2>), dim3(ring_grid), dim3(ring_block), 0, stream, a, b, c, m, n,
                           k, k_split, depth, out_ws, ctr);
    } else if (ring == MCHIP_RING_MID) {
        hipLaunchKernelGGL((matmul_ring_f32<RingMid, 2>), dim3(ring_grid), dim3(ring_block), 0, stream, a, b, c, m, n,
                           k, k_split, depth, out_ws, ctr);
    } else if (double_buffer) {
        if (vec) {
            hipLaunchKernelGGL((matmul_mfma_f32<true, true>), grid, dim3(256), 0, stream, a, b, c, m, n, k, k_split, out_ws);
        } else {
            hipLaunchKernelGGL((matmul_mfma_f32<true, false>), grid, dim3(256), 0, stream, a, b, c, m, n, k, k_split, out_ws);
        }
    } else {
        if (vec) {
            hipLaunchKernelGGL((matmul_mfma_f32<false, true>), grid, dim3(256), 0, stream, a, b, c, m, n, k, k_split, out_ws);
        } else {
            hipLaunchKernelGGL((matmul_mfma_f32<false, false>), grid, dim3(256), 0, stream, a, b, c, m, n, k, k_split, out_ws);
        }
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || depth == 1 || ctr != nullptr) return e;
    return mchip_sum_split_partials(workspace, c, static_cast<std::size_t>(m) * n, depth, stream);
}

}  // namespace

extern "C" int mchip_f32_ring_plan_cfg(int m, int n, int k, int depth, int cu_count, int cfg, unsigned* grid,
                                       unsigned* block) {
    *grid = 0;
    *block = 0;
    if (m < 1 || n < 4 || k < kRBKRing || k % kRBKRing != 0 || n % 4 != 0 || depth < 1 || cu_count < 1) {
        return MCHIP_RING_NONE;
    }
    // The ring's buffer loads and stores take 31-bit byte offsets from a
    // tile's origin: up to 256 rows of A, K + 32 rows of B and 256 rows of C
    // past it.
    if (256LL * k * 4 >= (1LL << 31) || (static_cast<long long>(k) + 32) * n * 4 >= (1LL << 31) ||
        256LL * n * 4 >= (1LL << 31)) {
        return MCHIP_RING_NONE;
    }
    if (cfg != MCHIP_RING_NONE) {
        // A forced configuration: its tiles, in persistent blocks (at most
        // one per CU for big, thin and wide8, two for wide and mid).
        long long bm = 0, bn = 0, per_cu = 1;
        unsigned threads = 0;
        switch (cfg) {
            case MCHIP_RING_BIG: bm = RingBig::kBM, bn = RingBig::kBN, threads = RingBig::kThreads; break;
            case MCHIP_RING_WIDE: bm = RingWide::kBM, bn = RingWide::kBN, threads = RingWide::kThreads, per_cu = 2; break;
            case MCHIP_RING_MID: bm = RingMid::kBM, bn = RingMid::kBN, threads = RingMid::kThreads, per_cu = 2; break;
            case MCHIP_RING_THIN: bm = RingThin::kBM, bn = RingThin::kBN, threads = RingThin::kThreads; break;
            case MCHIP_RING_WIDE8: bm = RingWide8::kBM, bn = RingWide8::kBN, threads = RingWide8::kThreads; break;
            default: return MCHIP_RING_NONE;
        }
        const long long units = ((m + bm - 1) / bm) * ((n + bn - 1) / bn) * depth;
        *grid = static_cast<unsigned>(std::min(units, per_cu * cu_count));
        *block = threads;
        return cfg;
    }
    // Time in units of one 128x128 tile-split on a whole CU: the tile-splits
    // of the busiest CU x work per tile-split (a 256x256 tile is four) /
    // efficiency. With the staged buffer-load fetch interleaved with the
    // MFMAs, wide runs 1-4% faster than big where both fill every CU (bare,
    // one MI355X: 8192^3 7528 against 7607 us, 4096^3 941 against 965,
    // 8192x2048x512 126.6 against 131.6, 2048x8192x2048 477 against 486).
    // With these factors the model never prefers big (a 256x256 tile round is
    // four 128x128 tile-splits on a CU either way); big stays for ring=big.
    const long long cus = cu_count;
    if (m <= RingThin::kBM) {
        const long long t32 = static_cast<long long>((n + 127) / 128) * depth;
        *grid = static_cast<unsigned>(std::min(t32, cus));
        *block = RingThin::kThreads;
        return MCHIP_RING_THIN;
    }
    const long long t256 = static_cast<long long>((m + 255) / 256) * ((n + 255) / 256) * depth;
    const long long t128 = static_cast<long long>((m + 127) / 128) * ((n + 127) / 128) * depth;
    const double big = static_cast<double>((t256 + cus - 1) / cus) * 4.0 / 0.92;
    const long long wide_grid = std::min(t128, 2 * cus);
    const double wide = static_cast<double>((wide_grid > cus ? 2 : 1) * ((t128 + wide_grid - 1) / wide_grid)) / 0.95;
    if (big <= wide) {
        *grid = static_cast<unsigned>(std::min(t256, cus));
        *block = RingBig::kThreads;
        return MCHIP_RING_BIG;
    }
    *grid = static_cast<unsigned>(wide_grid);
    if (t128 <= cus) {
        // One tile (or tile-split) per CU at most: the 8-wave block (two
        // waves per SIMD; 1024^3 in 4 splits 27.2 against 27.7 us).
        *block = RingWide8::kThreads;
        return MCHIP_RING_WIDE8;
    }
    *block = RingWide::kThreads;
    return MCHIP_RING_WIDE;
}

extern "C" int mchip_f32_ring_plan(int m, int n, int k, int depth, int cu_count, unsigned* grid, unsigned* block) {
    return mchip_f32_ring_plan_cfg(m, n, k, depth, cu_count, MCHIP_RING_NONE, grid, block);
}

extern "C" int mchip_narrow_rows(int shape) {
    return shape == MCHIP_NARROW_64X64 ? 64 : shape == MCHIP_NARROW_32X64 ? 32 : 16;
}

extern "C" int mchip_narrow_cols(int shape) {
    return shape == MCHIP_NARROW_16X32 ? 32 : 64;
}

extern "C" int mchip_f32_narrow_plan(int m, int n, int k, int max_splits, int cu_count, int force, int* shape,
                                     int* splits, int* k_split) {
    *shape = *splits = *k_split = 0;
    if (m < 1 || n < 4 || n % 4 != 0 || k < 16 || k % 16 != 0 || max_splits < 1 || cu_count < 1) return 0;
    // The narrow body's buffer loads take 31-bit byte offsets from a block's
    // origin: up to 64 rows of A and K + 16 rows of B past it.
    if (64LL * k * 4 >= (1LL << 31) || (static_cast<long long>(k) + 16) * n * 4 >= (1LL << 31)) return 0;
    auto tiles_of = [&](int sh) {
        return static_cast<long long>((m + mchip_narrow_rows(sh) - 1) / mchip_narrow_rows(sh)) *
               ((n + mchip_narrow_cols(sh) - 1) / mchip_narrow_cols(sh));
    };
    // Short K: the first tile shape that gives more than half the CUs a
    // tile runs unsplit, one block per CU with no partials and no sum
    // launch. Measured on an MI355X (launch plus sum, one operand set):
    // 256x512x2048 on 16x32 tiles 9.6 us against 11.2 on 32x64 tiles in 4
    // ranges; 512^3 on 16x64 tiles 5.4 against 8.3 on 32x64 unsplit;
    // 1024^3 on 64x64 tiles 19.6 us against 26.7 on the ring in 4 splits
    // (graph-timed, operands past the MALL). With
    // longer K the smaller tiles' extra operand traffic costs more than a
    // sum launch (256x256x16384: 32.6 us on 16x32 tiles in 2 ranges against
    // 24.8 on 32x64 in 8).
    // 64x64 tiles also run two per CU (in two rounds of one block per CU):
    // 1024x2048x512 22.6 us against 24.2 on the ring unsplit,
    // 1024x2048x1024 38.9 against 44.2 in 2 splits, 512x4096x1024 43.0
    // against 44.5; at four per CU the ring wins (2048x2048x512: 44.3
    // against 38.2).
    if (m > 16 && k <= 2048) {
        for (int sh : {MCHIP_NARROW_64X64, MCHIP_NARROW_32X64, MCHIP_NARROW_16X64, MCHIP_NARROW_16X32}) {
            const long long t = tiles_of(sh);
            const long long per_cu = sh == MCHIP_NARROW_64X64 ? 2 : 1;
            if (2 * t > cu_count && t <= per_cu * cu_count) {
                *shape = sh;
                *k_split = k;
                *splits = 1;
                return 1;
            }
        }
    }
    // 64x64 tiles when they need at most two K ranges (more than a quarter
    // of the CUs get a tile), else 32x64: deep K splits of the larger tile
    // gained nothing. Measured on an MI355X (graph-timed, operands past the
    // MALL, launch plus sum): 1024x1024x4096 unsplit on 64x64 65.1 us
    // against 73.7 on the ring (32x64 tiles would number 512);
    // 128x4096x4096 in 2 ranges 42.3 against 43.6 unsplit on 32x64;
    // 512x512x8192 in 4 ranges 39.8 against 39.3 in 2; 256x256x16384 in 16
    // ranges 23.0 against 23.0 in 8.
    const int sh = m <= 16                                             ? MCHIP_NARROW_16X64_STREAM
                   : m >= 64 && 4 * tiles_of(MCHIP_NARROW_64X64) > cu_count ? MCHIP_NARROW_64X64
                                                                           : MCHIP_NARROW_32X64;
    const long long tiles = tiles_of(sh);
    // Measured on an MI355X (one-matmul launches, operands past the MALL):
    // against the ring body, the narrow body wins while its tiles fit one
    // per CU (256x2048x512: 9.4 against 16.2 us; 256x512x2048 in 4 ranges
    // 13.0 against 16.4; 512^3 8.9 against 13.0; 1024x512x2048 25.9 against
    // 28.1; 16x4096x4096 in 4 ranges 17.2 against 20.6) and loses beyond
    // (1024^3 34.8 against 28.1; 1024x2048x512 33.7 against 28.8): its
    // tiles reuse each operand byte a third as often.
    if (!force && tiles > cu_count) return 0;
    // K ranges: the largest power of two that keeps tiles x ranges within
    // the CUs and each range at least 64 deep.
    int s = 1;
    while (s * 2 <= max_splits && tiles * s * 2 <= cu_count && k / (s * 2) >= 64) s *= 2;
    const int ks = ((k + s - 1) / s + 15) / 16 * 16;
    *shape = sh;
    *k_split = ks;
    *splits = (k + ks - 1) / ks;
    return 1;
}

extern "C" int mchip_launch_narrow(const float* a, const float* b, float* c, int m, int n, int k, void* stream,
                                   int splits, int rows, float* workspace) {
    if (m < 1 || n < 4 || n % 4 != 0 || k < 16 || k % 16 != 0 || splits < 1) return hipErrorInvalidValue;
    if ((rows != 16 && rows != 32) || (rows == 16 && m > 16)) return hipErrorInvalidValue;
    const int k_split = ((k + splits - 1) / splits + 15) / 16 * 16;
    return launch_narrow(a, b, c, m, n, k, static_cast<hipStream_t>(stream),
                         rows == 16 ? MCHIP_NARROW_16X64_STREAM : MCHIP_NARROW_32X64, k_split,
                         (k + k_split - 1) / k_split, workspace, nullptr);
}

extern "C" int mchip_sum_split_partials(const float* partial, float* c, size_t count, int splits, void* stream) {
    if (splits < 1) return hipErrorInvalidValue;
    hipStream_t s = static_cast<hipStream_t>(stream);
    // float4 lanes only when there are enough of them to fill the chip (four
    // waves per CU); else one float per lane, so more lanes share the loads.
    const std::size_t fill = static_cast<std::size_t>(std::max(device_cu_count(), 1)) * 256;
    const bool vec = count % 4 == 0 && aligned16(partial) && aligned16(c) && count / 4 >= fill;
    const std::size_t items = vec ? count / 4 : count;
    const unsigned blocks = static_cast<unsigned>(std::max<std::size_t>(1, std::min<std::size_t>((items + 255) / 256, 8192)));
    const int rest = splits - 1;  // loads after split 0's
    if (vec) {
        const f32x4* p = reinterpret_cast<const f32x4*>(partial);
        f32x4* o = reinterpret_cast<f32x4*>(c);
        if (rest <= 4) {
            hipLaunchKernelGGL((sum_splits_chunked<f32x4, 4>), dim3(blocks), dim3(256), 0, s, p, o, items, splits);
        } else if (rest <= 8) {
            hipLaunchKernelGGL((sum_splits_chunked<f32x4, 8>), dim3(blocks), dim3(256), 0, s, p, o, items, splits);
        } else {
            hipLaunchKernelGGL((sum_splits_chunked<f32x4, 16>), dim3(blocks), dim3(256), 0, s, p, o, items, splits);
        }
    } else if (rest <= 8) {
        hipLaunchKernelGGL((sum_splits_chunked<float, 8>), dim3(blocks), dim3(256), 0, s, partial, c, items, splits);
    } else if (rest <= 16) {
        hipLaunchKernelGGL((sum_splits_chunked<float, 16>), dim3(blocks), dim3(256), 0, s, partial, c, items, splits);
    } else if (rest <= 32) {
        hipLaunchKernelGGL((sum_splits_chunked<float, 32>), dim3(blocks), dim3(256), 0, s, partial, c, items, splits);
    } else {
        hipLaunchKernelGGL((sum_splits_chunked<float, 64>), dim3(blocks), dim3(256), 0, s, partial, c, items, splits);
    }
    return hipGetLastError();
}

extern "C" int mchip_launch_tensor_core(int kernel, const float* a, const float* b, float* c, int m, int n, int k,
                                        void* stream, int splits, float* workspace);

extern "C" int mchip_launch_matmul(int kernel, const float* a, const float* b, float* c, int m, int n, int k,
                                   void* stream, int splits, float* workspace) {
    if (m < 1 || n < 1 || k < 1) return hipErrorInvalidValue;
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (kernel) {
        case kNaive: {
            const dim3 grid((n + 15) / 16, (m + 15) / 16);
            hipLaunchKernelGGL(matmul_naive, grid, dim3(16, 16), 0, s, a, b, c, m, n, k);
            return hipGetLastError();
        }
        case kTiled: {
            const dim3 grid((n + kTile - 1) / kTile, (m + kTile - 1) / kTile);
            hipLaunchKernelGGL(matmul_tiled, grid, dim3(kTile, kTile), 0, s, a, b, c, m, n, k);
            return hipGetLastError();
        }
        case kRegisterTiled128: {
            const dim3 grid((n + 127) / 128, (m + 127) / 128);
            hipLaunchKernelGGL((matmul_register_tiled<128, 128, 8, 8, 8>), grid, dim3(256), 0, s, a, b, c, m, n, k);
            return hipGetLastError();
        }
        case kRegisterTiled64: {
            const dim3 grid((n + 63) / 64, (m + 63) / 64);
            hipLaunchKernelGGL((matmul_register_tiled<64, 64, 8, 4, 4>), grid, dim3(256), 0, s, a, b, c, m, n, k);
            return hipGetLastError();
        }
        case kVectorized: return launch_mfma_f32(false, a, b, c, m, n, k, s, 1, nullptr, MCHIP_RING_NONE, false);
        case kDoubleBuffered: return launch_mfma_f32(true, a, b, c, m, n, k, s, 1, nullptr, MCHIP_RING_NONE, false);
        case kSplitK: return launch_mfma_f32(true, a, b, c, m, n, k, s, splits, workspace, MCHIP_RING_NONE, true);
        case kTensorCoreTf32:
        case kTensorCoreBf16:
        case kTensorCoreF16: return mchip_launch_tensor_core(kernel, a, b, c, m, n, k, stream, splits, workspace);
        default: return hipErrorInvalidValue;  // Auto must be resolved first
    }
}

extern "C" int mchip_launch_matmul_cfg(int kernel, const float* a, const float* b, float* c, int m, int n, int k,
                                       void* stream, int splits, float* workspace, int ring_cfg) {
    if (ring_cfg == MCHIP_RING_NONE) return mchip_launch_matmul(kernel, a, b, c, m, n, k, stream, splits, workspace);
    if (m < 1 || n < 1 || k < 1) return hipErrorInvalidValue;
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (kernel) {
        case kDoubleBuffered:
            if (ring_cfg == MCHIP_RING_NARROW) return hipErrorInvalidValue;  // split_k only
            return launch_mfma_f32(true, a, b, c, m, n, k, s, 1, nullptr, ring_cfg, false);
        case kSplitK: return launch_mfma_f32(true, a, b, c, m, n, k, s, splits, workspace, ring_cfg, true);
        default: return hipErrorInvalidValue;  // only the ring rungs take a configuration
    }
}

extern "C" int mchip_matmul_k_ranges(int kernel, int m, int n, int k, int splits, int ring_cfg) {
    if (m < 1 || n < 1 || k < 1) return 0;
    switch (kernel) {
        case kSplitK: {
            const MfmaPlan p = plan_mfma_f32(true, true, true, true, true, true, m, n, k, splits, ring_cfg, true);
            return p.status == hipSuccess ? p.depth : 0;
        }
        case kTensorCoreBf16:
        case kTensorCoreF16: return mchip_tensor_core_k_ranges(k, splits);
        default: return 1;
    }
}

extern "C" unsigned long long mchip_split_counter_bytes(int m, int n) {
    if (m < 1 || n < 1) return 0;
    // The smallest tiles of any body that folds (16x32 narrow tiles).
    return 4ull * ((static_cast<unsigned long long>(m) + 15) / 16) * ((static_cast<unsigned long long>(n) + 31) / 32);
}

extern "C" int mchip_split_k_folds(int m, int n, int k, int splits, int ring_cfg) {
    if (m < 1 || n < 1 || k < 1) return 0;
    return plan_mfma_f32(true, true, true, true, true, true, m, n, k, splits, ring_cfg, true).can_fold() ? 1 : 0;
}

extern "C" int mchip_launch_matmul_fold(int kernel, const float* a, const float* b, float* c, int m, int n, int k,
                                        void* stream, int splits, float* workspace, int ring_cfg, unsigned* counters) {
    if (kernel != kSplitK || counters == nullptr) {
        return mchip_launch_matmul_cfg(kernel, a, b, c, m, n, k, stream, splits, workspace, ring_cfg);
    }
    if (m < 1 || n < 1 || k < 1) return hipErrorInvalidValue;
    return launch_mfma_f32(true, a, b, c, m, n, k, static_cast<hipStream_t>(stream), splits, workspace, ring_cfg, true,
                           counters);
}
