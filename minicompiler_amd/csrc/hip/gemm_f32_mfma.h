// FP32 matrix-core GEMM body for gfx950 (v_mfma_f32_32x32x2_f32), shared by
// the ahead-of-time kernels (matmul_fp32.hip, identity epilogue) and the
// GEMMs compiled at run time with a fused elementwise epilogue (the
// executable's generated source embeds this file). Self-contained: no
// standard or HIP headers, so hipRTC compiles it as is.
#pragma once

typedef float mc_gemm_f32x4 __attribute__((ext_vector_type(4)));
typedef float mc_gemm_f32x16 __attribute__((ext_vector_type(16)));

// The identity epilogue: C[i] = the accumulated dot product.
struct McGemmStore {
    __device__ __forceinline__ float operator()(float v, unsigned) const { return v; }
};

// Block tile 128x128, K step 32, 256 lanes = 4 waves in a 2x2 grid, each wave
// a 64x64 quadrant as 2x2 v_mfma_f32_32x32x2_f32 accumulators (64 VGPRs).
//
// LDS: A row-major (k contiguous, row pitch 36 floats), B row-major (n
// contiguous, pitch 132). With 36-float rows, eight lanes reading 16 bytes
// each from eight consecutive rows touch 32 distinct banks.
//
// MFMA operand order. One v_mfma_f32_32x32x2_f32 multiplies a 32x2 slice of A
// by a 2x32 slice of B: lane l supplies row/column l % 32 and k slot l / 32.
// The result does not depend on which K index each (step, slot) pair stands
// for, as long as A and B use the same pairing; step s, slot h here stands
// for k = 16h + s of the 32-wide tile, so a lane reads its A values as four
// 16-byte vectors.
//
// Accumulator layout (32x32 result, 16 floats per lane): value v of lane l is
// row 8 (v / 4) + 4 (l / 32) + v % 4, column l % 32.

constexpr int kMBM = 128, kMBN = 128, kMBK = 32;
constexpr int kAPitch = kMBK + 4;
constexpr int kBPitch = kMBN + 4;

// 4 consecutive floats of a row-major matrix (leading dimension ld) from
// (row, col); zeros at or past row_end / col_end. kVec: one 16-byte load
// (rows 16-byte aligned and col_end a multiple of 4).
template <bool kVec>
__device__ __forceinline__ mc_gemm_f32x4 mc_gemm_load4(const float* __restrict__ p, int row, int col, int row_end, int col_end,
                                       int ld) {
    mc_gemm_f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
    if (row >= row_end) return v;
    const float* s = p + static_cast<long long>(row) * ld + col;
    if constexpr (kVec) {
        if (col < col_end) v = *reinterpret_cast<const mc_gemm_f32x4*>(s);
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            if (col + e < col_end) v[e] = s[e];
        }
    }
    return v;
}

// The block's tile of C (grid: x over N, y over M, z over K splits). With one
// split the epilogue maps each accumulated value v of element i = row n + col
// to what is stored; with several, the raw partial sums go to `partial` and
// the epilogue is applied where the splits are summed.
template <bool kDouble, bool kVec, typename Epilogue>
__device__ __forceinline__ void mc_gemm_f32_mfma(const float* __restrict__ a, const float* __restrict__ b,
                                                 float* __restrict__ c, int m, int n, int k, int k_split,
                                                 float* __restrict__ partial, const Epilogue& epilogue) {
    constexpr int S = kDouble ? 2 : 1;
    __shared__ __attribute__((aligned(16))) float as[S][kMBM][kAPitch];
    __shared__ __attribute__((aligned(16))) float bs[S][kMBK][kBPitch];

    const int tid = threadIdx.x;
    const int wave = tid / 64, lane = tid % 64;
    const int wr = (wave / 2) * 64, wc = (wave % 2) * 64;
    const int half = lane / 32, li = lane % 32;
    const int row0 = blockIdx.y * kMBM, col0 = blockIdx.x * kMBN;
    const int kb = blockIdx.z * k_split;
    const int ke = k < kb + k_split ? k : kb + k_split;

    mc_gemm_f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = mc_gemm_f32x16{};

    // Per tile: A is 128 rows x 8 vectors, B 32 rows x 32 vectors; 4 of each per lane.
    mc_gemm_f32x4 ra[4], rb[4];
    auto global_load = [&](int k0) {
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const int f = tid + l * 256;
            ra[l] = mc_gemm_load4<kVec>(a, row0 + f / 8, k0 + (f % 8) * 4, m, ke, k);
            rb[l] = mc_gemm_load4<kVec>(b, k0 + f / 32, col0 + (f % 32) * 4, ke, n, n);
        }
    };
    auto lds_store = [&](int s) {
#pragma unroll
        for (int l = 0; l < 4; ++l) {
            const int f = tid + l * 256;
            *reinterpret_cast<mc_gemm_f32x4*>(&as[s][f / 8][(f % 8) * 4]) = ra[l];
            *reinterpret_cast<mc_gemm_f32x4*>(&bs[s][f / 32][(f % 32) * 4]) = rb[l];
        }
    };
    auto multiply = [&](int s) {
#pragma unroll
        for (int q = 0; q < kMBK / 8; ++q) {
            mc_gemm_f32x4 av[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) av[i] = *reinterpret_cast<const mc_gemm_f32x4*>(&as[s][wr + i * 32 + li][half * 16 + q * 4]);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int kk = half * 16 + q * 4 + e;
                float bv[2];
#pragma unroll
                for (int j = 0; j < 2; ++j) bv[j] = bs[s][kk][wc + j * 32 + li];
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[i][e], bv[j], acc[i][j], 0, 0, 0);
            }
        }
    };

    const int tiles = ke > kb ? (ke - kb + kMBK - 1) / kMBK : 0;
    if constexpr (kDouble) {
        if (tiles > 0) {
            global_load(kb);
            lds_store(0);
        }
        __syncthreads();
        for (int t = 0; t < tiles; ++t) {
            const int cur = t & 1;
            const bool more = t + 1 < tiles;
            if (more) global_load(kb + (t + 1) * kMBK);
            multiply(cur);
            // The other stage was last read before the previous barrier.
            if (more) lds_store(cur ^ 1);
            __syncthreads();
        }
    } else {
        for (int t = 0; t < tiles; ++t) {
            global_load(kb + t * kMBK);
            __syncthreads();  // every wave is done with the previous tile
            lds_store(0);
            __syncthreads();
            multiply(0);
        }
    }

    const bool split = gridDim.z > 1;
    float* __restrict__ out = split ? partial + static_cast<long long>(blockIdx.z) * m * n : c;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int col = col0 + wc + j * 32 + li;
            if (col >= n) continue;
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int row = row0 + wr + i * 32 + 8 * (v / 4) + 4 * half + (v % 4);
                if (row >= m) continue;
                const long long at = static_cast<long long>(row) * n + col;
                out[at] = split ? acc[i][j][v] : epilogue(acc[i][j][v], static_cast<unsigned>(at));
            }
        }
    }
}

