// FP32 GEMM body for narrow tiles: C tiles of 16 kRG rows x 64 columns on
// v_mfma_f32_16x16x4f32, for products too small or too thin to fill the chip
// with the ring body's 128x128 and 256x256 tiles (M <= 16, where B is read
// once and HBM is the bound; and products of a few million outputs or
// fewer, where small tiles give every CU a share without deep K splits).
// Shared by the ahead-of-time kernels (identity epilogue) and the GEMMs
// compiled at run time with a fused elementwise epilogue. Self-contained (no
// headers), so hipRTC compiles it as is.
//
// No LDS staging of operands: each wave loads its A and B fragments straight
// from global memory (L2 for data other waves share) into registers, all the
// loads of a batch of K before the batch's MFMAs, so a wave keeps many loads
// in flight and each group's MFMAs start as soon as that group has landed.
//
// Decomposition: block (x, y, z) owns columns 64 x .. 64 x + 63, rows
// 16 kRG z .., and the y-th of `depth` ranges of K (k_split each); its kW
// waves cut that range into consecutive pieces, one accumulator set each.
// Lane l of a wave has k slot s = l / 16 and index c = l % 16. For each group
// of 16 k from kg the lane loads
//   A[16 r + c][kg + 4s .. kg + 4s + 3]          for row group r < kRG
//   B[kg + 4s + e][col0 + 4c .. col0 + 4c + 3]   for e = 0..3
// and MFMA (r, e, j) takes A load r's element e and B load e's element j:
// its k slot s is k = kg + 4s + e and its column slot c is column
// col0 + 4c + j, so accumulator (r, j) holds, in lane l, C[16 r + 4s + v]
// [col0 + 4c + j] for v = 0..3. The waves' tiles are then added in wave
// order through LDS (a fixed order), and the block stores its tile to C
// through the epilogue, or, with several K ranges, to its range's partial
// (summed afterwards in range order, the epilogue applied there).
//
// Requirements (checked by the host): k and k_split multiples of 16, n a
// multiple of 4, A and B 16-byte aligned (C and the partials may be at any
// float address). Rows past m read
// row m - 1 and columns past n the last column chunk (every load in
// bounds); what they produce is not stored.
#pragma once

typedef float mc_nw_f32x4 __attribute__((ext_vector_type(4)));

template <int N>
struct McNarrowUnits {
    static constexpr int value = N;
};

// A configuration: kRG row groups of 16, kW waves, kU groups of 16 k per
// batch of loads; kStreamB: B is read by one tile row only (M <= 16), so
// its loads are non-temporal (a read-only stream reached 7.1 TB/s with them
// against 6.3 TB/s without on an MI355X).
template <int kRG_, int kW_, int kU_, bool kStreamB_>
struct McNarrowCfg {
    static constexpr int kRG = kRG_, kW = kW_, kU = kU_;
    static constexpr bool kStreamB = kStreamB_;
    static constexpr int kRows = 16 * kRG, kCols = 64, kThreads = 64 * kW;
};

// The configurations the library runs: 16-row tiles (M <= 16: one batch
// covers a wave's whole K range at the planner's splits) and 32-row tiles.
using McNarrow16 = McNarrowCfg<1, 4, 8, true>;
using McNarrow32 = McNarrowCfg<2, 4, 4, false>;

// The tile of C at (row0, col0) and its K range [kb, ke), accumulated by
// this block; the epilogue maps each value v of flat element i to what is
// stored (out = C), or the raw sums go to `out` (a partial).
template <class Cfg, typename Epilogue>
__device__ __forceinline__ void mc_gemm_f32_narrow(const float* __restrict__ a, const float* __restrict__ b,
                                                   float* __restrict__ c, int m, int n, int k, int k_split,
                                                   int depth, float* __restrict__ partial, const Epilogue& epilogue) {
    constexpr int kRG = Cfg::kRG, kW = Cfg::kW;
    __shared__ mc_nw_f32x4 red[kW][Cfg::kRows][16];  // [wave][row][column chunk]
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    const int s = lane >> 4, cl = lane & 15;
    const int col0 = blockIdx.x * Cfg::kCols;
    const int row0 = blockIdx.z * Cfg::kRows;
    const int colc = col0 + 4 * cl < n ? col0 + 4 * cl : n - 4;

    // This wave's K range: the block's range cut into kW pieces of whole
    // 16-k groups (the last pieces may be empty).
    const int kb = blockIdx.y * k_split;
    const int ke = kb + k_split < k ? kb + k_split : k;
    const int groups = (ke - kb) / 16;
    const int per = (groups + kW - 1) / kW;
    const int g0 = wave * per < groups ? wave * per : groups;
    const int g1 = g0 + per < groups ? g0 + per : groups;

    const float* __restrict__ ap[kRG];
#pragma unroll
    for (int r = 0; r < kRG; ++r) {
        const int row = row0 + 16 * r + cl < m ? row0 + 16 * r + cl : m - 1;
        ap[r] = a + static_cast<long long>(row) * k + kb + 4 * s;
    }
    const float* __restrict__ bp = b + static_cast<long long>(kb + 4 * s) * n + colc;
    const long long nn = n;

    mc_nw_f32x4 acc[kRG][4] = {};
    // kU groups of 16 k from group g, straight-line: every load first, then
    // the MFMAs, each waiting only for its own group's loads.
    auto batch = [&](int g, auto units) {
        constexpr int kU = decltype(units)::value;
        mc_nw_f32x4 av[kU][kRG];
        mc_nw_f32x4 bv[kU][4];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
#pragma unroll
            for (int r = 0; r < kRG; ++r) av[u][r] = *reinterpret_cast<const mc_nw_f32x4*>(ap[r] + 16 * (g + u));
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const mc_nw_f32x4* p = reinterpret_cast<const mc_nw_f32x4*>(bp + (16LL * (g + u) + e) * nn);
                if constexpr (Cfg::kStreamB) {
                    bv[u][e] = __builtin_nontemporal_load(p);
                } else {
                    bv[u][e] = *p;
                }
            }
        }
        // Left to itself the scheduler interleaves each load with the MFMAs
        // that use it and waits for it there: one load in flight.
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < kU; ++u)
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int r = 0; r < kRG; ++r)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        acc[r][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[u][r][e], bv[u][e][j], acc[r][j], 0, 0, 0);
    };
    int g = g0;
    for (; g + Cfg::kU <= g1; g += Cfg::kU) batch(g, McNarrowUnits<Cfg::kU>{});
    for (; g < g1; ++g) batch(g, McNarrowUnits<1>{});

    // Lane l holds rows 16 r + 4s + v of column chunk cl.
#pragma unroll
    for (int r = 0; r < kRG; ++r)
#pragma unroll
        for (int v = 0; v < 4; ++v)
            red[wave][16 * r + 4 * s + v][cl] = mc_nw_f32x4{acc[r][0][v], acc[r][1][v], acc[r][2][v], acc[r][3][v]};
    __syncthreads();
    // The tile's chunks, summed over the waves in wave order.
    const bool raw = depth > 1;
    float* __restrict__ out = raw ? partial + static_cast<long long>(blockIdx.y) * m * n : c;
    // C or a partial may sit at any 4-byte address (a caller's workspace):
    // then the chunk is stored as four floats, the same values.
    const bool vec_out = (reinterpret_cast<unsigned long long>(out) & 15) == 0;
    for (int t = threadIdx.x; t < Cfg::kRows * 16; t += Cfg::kThreads) {
        const int r = t >> 4, ch = t & 15;
        mc_nw_f32x4 sum = red[0][r][ch];
#pragma unroll
        for (int w = 1; w < kW; ++w) sum += red[w][r][ch];
        const int row = row0 + r, col = col0 + 4 * ch;
        if (row < m && col < n) {
            const long long at = static_cast<long long>(row) * n + col;
            if (!raw) {
#pragma unroll
                for (int j = 0; j < 4; ++j) sum[j] = epilogue(sum[j], static_cast<unsigned>(at + j));
            }
            if (vec_out) {
                *reinterpret_cast<mc_nw_f32x4*>(out + at) = sum;
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) out[at + j] = sum[j];
            }
        }
    }
}
