// bf16 / fp16 matrix-core matmul for gfx950 (v_mfma_f32_16x16x32_bf16 and
// _f16), FP32 accumulation and output. Takes the place of the reference's
// tensor-core kernels (src/cuda/matmul_tensor_core.cu:96-297):
//   - fp32 inputs rounded to nearest-even into bf16 / fp16 as they are
//     staged into LDS (the reference's mode), or
//   - inputs already in bf16 / fp16 in device memory (the pre-cast mode).
// TF32 does not exist on gfx950 (no xf32 matrix instruction): those requests
// report hipErrorNotSupported.
//
// Block tile 128x128, K step 64, 256 lanes = 4 waves in a 2x2 grid, each wave
// a 64x64 quadrant as 4x4 16x16 accumulators. A is staged row-major
// (k contiguous), B transposed (n-major, k contiguous), so each lane's MFMA
// operand is one 16-byte LDS read. Two LDS stages; split-K as in the FP32
// kernels.
//
// v_mfma_f32_16x16x32_*: lane l supplies row (A) / column (B) l % 16 and
// eight k values from group l / 16; A and B use the same k assignment, so
// any assignment gives the same sum (here group g holds k = 8g .. 8g+7 of the
// 32-wide step). Result: value v of lane l is row 4 (l / 16) + v, column l % 16.

#include "matmul.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstddef>
#include <cstdint>

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned short u16x4 __attribute__((ext_vector_type(4)));
typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

enum { kTensorCoreTf32 = 8, kTensorCoreBf16 = 9, kTensorCoreF16 = 10 };

// Round-to-nearest-even of a float to the upper 16 bits (bf16). NaN stays a
// quiet NaN; values that round past the largest finite bf16 become infinity.
__device__ __forceinline__ unsigned short to_bf16_bits(float x) {
    const unsigned u = __float_as_uint(x);
    if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<unsigned short>((u >> 16) | 0x0040u);
    const unsigned rounded = u + 0x7fffu + ((u >> 16) & 1u);
    return static_cast<unsigned short>(rounded >> 16);
}

// IEEE half, round to nearest even (the hardware conversion).
__device__ __forceinline__ unsigned short to_f16_bits(float x) {
    const _Float16 h = static_cast<_Float16>(x);
    return __builtin_bit_cast(unsigned short, h);
}

template <bool kBf16>
__device__ __forceinline__ unsigned short to_bits(float x) {
    if constexpr (kBf16) return to_bf16_bits(x);
    return to_f16_bits(x);
}

template <bool kBf16>
__device__ __forceinline__ f32x4 mfma(u16x8 a, u16x8 b, f32x4 c) {
    if constexpr (kBf16) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                       c, 0, 0, 0);
    } else {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                      0, 0, 0);
    }
}

constexpr int kBM = 128, kBN = 128, kBK = 64;
constexpr int kPitch = kBK + 8;  // halves per LDS row: 144 bytes, keeps 16-byte alignment

// Element source: fp32 in memory (rounded here) or 16-bit already.
template <bool kBf16, bool kF32In>
struct Source {
    using T = typename std::conditional<kF32In, float, unsigned short>::type;
};

// Four consecutive elements as 16-bit patterns; zeros out of range.
template <bool kBf16, bool kF32In, bool kVec>
__device__ __forceinline__ u16x4 load4(const void* __restrict__ base, int row, int col, int row_end, int col_end,
                                       int ld) {
    u16x4 v = {0, 0, 0, 0};
    if (row >= row_end) return v;
    if constexpr (kF32In) {
        const float* s = static_cast<const float*>(base) + static_cast<std::ptrdiff_t>(row) * ld + col;
        if constexpr (kVec) {
            if (col < col_end) {
                const f32x4 f = *reinterpret_cast<const f32x4*>(s);
                v = u16x4{to_bits<kBf16>(f.x), to_bits<kBf16>(f.y), to_bits<kBf16>(f.z), to_bits<kBf16>(f.w)};
            }
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (col + e < col_end) v[e] = to_bits<kBf16>(s[e]);
            }
        }
    } else {
        const unsigned short* s =
            static_cast<const unsigned short*>(base) + static_cast<std::ptrdiff_t>(row) * ld + col;
        if constexpr (kVec) {
            if (col < col_end) v = *reinterpret_cast<const u16x4*>(s);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (col + e < col_end) v[e] = s[e];
            }
        }
    }
    return v;
}

template <bool kBf16, bool kF32In, bool kVec>
__global__ void __launch_bounds__(256, 2) matmul_mfma16(const void* __restrict__ a, const void* __restrict__ b,
                                                        float* __restrict__ c, int m, int n, int k, int k_split,
                                                        float* __restrict__ partial) {
    __shared__ __attribute__((aligned(16))) unsigned short as[2][kBM][kPitch];
    __shared__ __attribute__((aligned(16))) unsigned short bt[2][kBN][kPitch];

    const int tid = threadIdx.x;
    const int wave = tid / 64, lane = tid % 64;
    const int wr = (wave / 2) * 64, wc = (wave % 2) * 64;
    const int g = lane / 16, li = lane % 16;
    const int row0 = blockIdx.y * kBM, col0 = blockIdx.x * kBN;
    const int kb = blockIdx.z * k_split;
    const int ke = min(k, kb + k_split);

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // A tile: 128 rows x 16 quads; B tile: 64 rows x 32 quads. 8 of each per lane.
    u16x4 ra[8], rb[8];
    auto global_load = [&](int k0) {
#pragma unroll
        for (int l = 0; l < 8; ++l) {
            const int f = tid + l * 256;
            ra[l] = load4<kBf16, kF32In, kVec>(a, row0 + f / 16, k0 + (f % 16) * 4, m, ke, k);
            rb[l] = load4<kBf16, kF32In, kVec>(b, k0 + f / 32, col0 + (f % 32) * 4, ke, n, n);
        }
    };
    auto lds_store = [&](int s) {
#pragma unroll
        for (int l = 0; l < 8; ++l) {
            const int f = tid + l * 256;
            *reinterpret_cast<u16x4*>(&as[s][f / 16][(f % 16) * 4]) = ra[l];
            const int kk = f / 32, cc = (f % 32) * 4;
#pragma unroll
            for (int e = 0; e < 4; ++e) bt[s][cc + e][kk] = rb[l][e];
        }
    };
    auto multiply = [&](int s) {
#pragma unroll
        for (int q = 0; q < kBK / 32; ++q) {
            u16x8 av[4], bv[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) av[i] = *reinterpret_cast<const u16x8*>(&as[s][wr + i * 16 + li][q * 32 + g * 8]);
#pragma unroll
            for (int j = 0; j < 4; ++j) bv[j] = *reinterpret_cast<const u16x8*>(&bt[s][wc + j * 16 + li][q * 32 + g * 8]);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = mfma<kBf16>(av[i], bv[j], acc[i][j]);
        }
    };

    const int tiles = ke > kb ? (ke - kb + kBK - 1) / kBK : 0;
    if (tiles > 0) {
        global_load(kb);
        lds_store(0);
    }
    __syncthreads();
    for (int t = 0; t < tiles; ++t) {
        const int cur = t & 1;
        const bool more = t + 1 < tiles;
        if (more) global_load(kb + (t + 1) * kBK);
        multiply(cur);
        if (more) lds_store(cur ^ 1);
        __syncthreads();
    }

    float* __restrict__ out = gridDim.z == 1 ? c : partial + static_cast<std::ptrdiff_t>(blockIdx.z) * m * n;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int col = col0 + wc + j * 16 + li;
            if (col >= n) continue;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int row = row0 + wr + i * 16 + 4 * g + v;
                if (row < m) out[static_cast<std::ptrdiff_t>(row) * n + col] = acc[i][j][v];
            }
        }
    }
}

// ---------------------------------------------------------------- fast path
//
// 16-bit inputs already in HBM, K a multiple of 64, N a multiple of 8, rows
// 16-byte aligned. Block tile 256x256, 512 lanes = 8 waves in a 2x4 grid
// (two waves per SIMD), each wave a 128x64 quadrant as 8x4 accumulators of
// v_mfma_f32_16x16x32 (128 fp32 per lane, in AGPRs). One block per CU; the
// two waves of a SIMD hide each other's LDS and barrier waits.
//
// K is walked in steps of 32 through a ring of four 32 KiB LDS stages, with
// the two waves of each SIMD in ping-pong: waves 0-3 and waves 4-7 run the
// same sequence one phase apart, alternating a memory phase (issue the
// global -> LDS fetch of step t+3, read step t's operands from LDS into
// registers) and a compute phase (step t's 32 MFMAs), so each SIMD's matrix
// unit is fed by one wave while the other loads. Phases are separated by a
// plain s_barrier of all 8 waves (no memory fence: a fence would also wait
// for the fetches still in flight); a memory phase ends with a wait for this
// wave's fetch of step t+1 and for its LDS reads.
//
// Global -> LDS without registers: global_load_lds_dwordx4 writes lane l's
// 16 bytes at (LDS base + 16 l), so one wave instruction fills 1 KiB of LDS;
// the swizzles below are applied by choosing which global chunk each lane
// fetches. Rows and columns past the matrix edge are clamped to the last row
// / column chunk, so every fetch is in bounds; the values they bring only
// reach C rows or columns that are not stored.
//
// LDS layout of a stage (bytes):
//   A [16 blocks of 16 rows][4 chunks of 8 k][16 rows], at 0: chunk c of
//     row r at 1024 (r / 16) + 256 c + 16 (r % 16). A fragment read (16 rows
//     x one chunk per 16 lanes, ds_read_b128) is then 1 KiB read linearly
//     (lane l at 16 l), which gfx950 serves without bank conflicts; row-major
//     rows with any chunk swizzle measured 4 conflict cycles per read. One
//     fetch instruction still covers 16 whole rows (64 bytes each).
//   B [32 k rows][32 chunks of 8 n], at 16 KiB: k row kr at 512 kr; logical
//     chunk c stored at chunk c ^ 2 tb(kr), tb(kr) = (kr & 3) | ((kr >> 3) & 3) << 2,
//     i.e. 32-byte pairs XOR tb. B stays n-contiguous and is read with
//     ds_read_b64_tr_b16: within each 16 lanes, lane 4e + c supplies the
//     address of 4 values (row e, columns 4c..4c+3) and lane i receives
//     column i of rows 0..3. Two such reads give a lane the 8 consecutive k
//     of one column that the MFMA B operand needs. The 16 rows one read
//     instruction touches fall in distinct 32-byte bank windows.
//
// The MFMA is issued with the B fragment as its first operand and the A
// fragment as its second, which yields C^T tiles: value v of lane l is
// C[m0 + l % 16][n0 + 4 (l / 16) + v], four consecutive columns, stored as
// one 16-byte write.
//
// Tiles are handed out in row-major order. The 256 blocks resident at a time
// then cover a band of a few tile rows across all of N: A's band and all of
// B (160 MiB at 8192^3) stay inside the 256 MiB MALL, and each XCD (block b
// runs on XCD b % 8) holds every eighth tile column of the band. Measured
// against grouped and XCD-remapped orders (A and B panels shared inside one
// XCD's L2, but the XCDs spread over all of A), row-major was as fast or
// faster at 8192^3.

typedef short s16x4 __attribute__((ext_vector_type(4)));
#define MC_LDS __attribute__((address_space(3)))

constexpr int kFBM = 256, kFBN = 256, kFBK = 32;
constexpr int kFThreads = 512;
constexpr int kFWaves = kFThreads / 64;
constexpr int kFStages = 4;
constexpr int kFStage = 32 * 1024;
constexpr int kFBOffset = 16 * 1024;
constexpr int kFRowFrags = 8;  // 16-row A fragments per wave (128 rows)
constexpr int kFColFrags = 4;  // 16-column B fragments per wave (64 columns)
// global_load_lds instructions per wave per step: 2 for A, 2 for B.
constexpr int kFFetchPerStep = 4;

__device__ __forceinline__ int swz_b(int kr) { return (kr & 3) | (((kr >> 3) & 3) << 2); }

// Per-lane addressing, set up once per block.
struct FastLane {
    const unsigned short* a_src[2];  // A chunk this lane fetches per instruction (k offset 0)
    const unsigned short* b_src[2];  // B chunk (k row offset 0)
    std::ptrdiff_t b_step;           // elements between consecutive K steps of B
    int a_off[kFRowFrags];           // LDS byte offsets of the A fragments
    int b_off[2][kFColFrags];        // LDS byte offsets of the two transposed B reads
    int wave;
};

__device__ __forceinline__ void fast_fetch(MC_LDS unsigned char* wr, const FastLane& L, int fetch_k) {
    MC_LDS unsigned char* sa = wr + L.wave * 32 * 64;
    MC_LDS unsigned char* sb = wr + kFBOffset + L.wave * 4 * 512;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        __builtin_amdgcn_global_load_lds(static_cast<const void*>(L.a_src[i] + fetch_k),
                                         reinterpret_cast<MC_LDS void*>(sa + i * 1024), 16, 0, 0);
    }
    const std::ptrdiff_t bk = (fetch_k / kFBK) * L.b_step;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        __builtin_amdgcn_global_load_lds(static_cast<const void*>(L.b_src[i] + bk),
                                         reinterpret_cast<MC_LDS void*>(sb + i * 1024), 16, 0, 0);
    }
}

__device__ __forceinline__ u16x8 fast_read_a(const MC_LDS unsigned char* rd, const FastLane& L, int f) {
    return *reinterpret_cast<const MC_LDS u16x8*>(rd + L.a_off[f]);
}

__device__ __forceinline__ u16x8 fast_read_b(const MC_LDS unsigned char* rd, const FastLane& L, int f) {
    MC_LDS unsigned char* p = const_cast<MC_LDS unsigned char*>(rd);
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(reinterpret_cast<MC_LDS s16x4*>(p + L.b_off[0][f]));
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(reinterpret_cast<MC_LDS s16x4*>(p + L.b_off[1][f]));
    return __builtin_bit_cast(u16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

// Memory phase: fetch step `fetch_k` into `wr` and read the operands of the
// step held in `rd` into (av, bv). `rd` and `wr` are distinct stages;
// declaring them __restrict__ gives the LDS reads alias scopes that keep the
// compiler from making them wait for the fetch.
__device__ __forceinline__ void fast_memory_phase(const MC_LDS unsigned char* __restrict__ rd,
                                                  MC_LDS unsigned char* __restrict__ wr, const FastLane& L, int fetch_k,
                                                  u16x8 (&av)[kFRowFrags], u16x8 (&bv)[kFColFrags]) {
    fast_fetch(wr, L, fetch_k);
#pragma unroll
    for (int f = 0; f < kFRowFrags; ++f) av[f] = fast_read_a(rd, L, f);
#pragma unroll
    for (int f = 0; f < kFColFrags; ++f) bv[f] = fast_read_b(rd, L, f);
}

// A workgroup barrier without a memory fence; the compiler may not move
// memory operations or MFMAs across it.
__device__ __forceinline__ void step_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

template <bool kBf16>
__global__ void __launch_bounds__(kFThreads, 1) matmul_mfma16_fast(const unsigned short* __restrict__ a,
                                                                   const unsigned short* __restrict__ b,
                                                                   float* __restrict__ c, int m, int n, int k) {
    __shared__ __attribute__((aligned(1024))) unsigned char smem[kFStages * kFStage];
    MC_LDS unsigned char* lds = (MC_LDS unsigned char*)(smem);  // generic -> LDS address space

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;

    // Tile of this block (row-major).
    const int tiles_n = (n + kFBN - 1) / kFBN;
    const int tm = static_cast<int>(blockIdx.x) / tiles_n, tn = static_cast<int>(blockIdx.x) % tiles_n;
    const int row0 = tm * kFBM, col0 = tn * kFBN;

    FastLane L;
    L.wave = wave;
    // A: wave w fills the 16-row blocks 2 w and 2 w + 1, one per
    // instruction; lane -> (row 32 w + 16 i + l % 16, chunk l / 16).
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int r = wave * 32 + i * 16 + (lane & 15);
        const int gr = min(row0 + r, m - 1);
        L.a_src[i] = a + static_cast<std::ptrdiff_t>(gr) * k + (lane >> 4) * 8;
    }
    // B: wave w fills k rows 4 w .. 4 w + 3, two per instruction; lane ->
    // (k row 4 w + 2 i + l / 32, physical chunk l % 32).
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int kr = wave * 4 + i * 2 + (lane >> 5);
        const int lc = (lane & 31) ^ (2 * swz_b(kr));
        const int gc = min(col0 + lc * 8, n - 8);
        L.b_src[i] = b + static_cast<std::ptrdiff_t>(kr) * n + gc;
    }
    L.b_step = static_cast<std::ptrdiff_t>(kFBK) * n;
    // Wave (wm, wn) of the 2x4 grid owns rows 128 wm .., columns 64 wn ...
    const int wr = (wave >> 2) * 128, wc = (wave & 3) * 64;
    const int li = lane & 15, g = lane >> 4;
#pragma unroll
    for (int f = 0; f < kFRowFrags; ++f) L.a_off[f] = (wr + f * 16) * 64 + lane * 16;
    // Transposed B reads: lane (g, e = (l % 16) / 4, cc = l % 4) points at
    // k row 8 g + 4 h + e, columns n0 + 4 cc .. + 3.
    const int te = (lane & 15) >> 2, tc = lane & 3;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int f = 0; f < kFColFrags; ++f) {
            const int kr = 8 * g + 4 * h + te;
            const int ncol = wc + f * 16 + 4 * tc;
            const int chunk = (ncol >> 3) ^ (2 * swz_b(kr));
            L.b_off[h][f] = kFBOffset + kr * 512 + (chunk << 4) + ((ncol & 4) << 1);
        }

    f32x4 acc[kFRowFrags][kFColFrags];
#pragma unroll
    for (int i = 0; i < kFRowFrags; ++i)
#pragma unroll
        for (int j = 0; j < kFColFrags; ++j) acc[i][j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    const int steps = k / kFBK;
    auto stage = [&](int t) { return lds + (t & (kFStages - 1)) * kFStage; };
    u16x8 av[kFRowFrags], bv[kFColFrags];
    // Prologue: steps 0..2 landed.
    const int pre = min(steps, kFStages - 1);
    for (int t = 0; t < pre; ++t) fast_fetch(stage(t), L, t * kFBK);
    __builtin_amdgcn_s_waitcnt(0);
    step_barrier();
    // Waves 4-7 start one phase late.
    const bool late = wave >= kFWaves / 2;
    if (late) step_barrier();

    // Every memory phase fetches: past the last step it fetches the last step
    // again, into the stage of step t-1, which no wave reads any more. After
    // the fetch of step t+3 this wave has the fetches of steps t+1..t+3 in
    // flight and waits for the oldest, which the other group reads two
    // phases later.
    const int last = (steps - 1) * kFBK;
    for (int t = 0; t < steps; ++t) {
        fast_memory_phase(stage(t), stage(t + 3), L, min((t + 3) * kFBK, last), av, bv);
        __builtin_amdgcn_s_waitcnt(0x0070 | (2 * kFFetchPerStep));  // vmcnt(8), lgkmcnt(0)
        step_barrier();
#pragma unroll
        for (int fi = 0; fi < kFRowFrags; ++fi)
#pragma unroll
            for (int fj = 0; fj < kFColFrags; ++fj) acc[fi][fj] = mfma<kBf16>(bv[fj], av[fi], acc[fi][fj]);
        step_barrier();
    }
    if (!late) step_barrier();
    __builtin_amdgcn_s_waitcnt(0);

    // acc[fi][fj] holds C[row0 + wr + 16 fi + l % 16][col0 + wc + 16 fj + 4 (l / 16) + v].
#pragma unroll
    for (int fi = 0; fi < kFRowFrags; ++fi) {
        const int row = row0 + wr + fi * 16 + li;
        if (row >= m) continue;
        float* crow = c + static_cast<std::ptrdiff_t>(row) * n;
#pragma unroll
        for (int fj = 0; fj < kFColFrags; ++fj) {
            const int col = col0 + wc + fj * 16 + 4 * g;
            if (col < n) *reinterpret_cast<f32x4*>(crow + col) = acc[fi][fj];
        }
    }
}

// The fast path takes 16-bit A and B with K a multiple of 64, N a multiple
// of 8 (every 16-byte B chunk wholly inside or outside a row), A, B and C
// 16-byte aligned, and no split.
bool fast_eligible(const void* a, const void* b, const float* c, int m, int n, int k, int splits) {
    const auto al = [](const void* p) { return reinterpret_cast<std::uintptr_t>(p) % 16 == 0; };
    return splits <= 1 && k % (2 * kFBK) == 0 && n % 8 == 0 && al(a) && al(b) && al(c) && m >= 1 && n >= 8;
}

template <bool kBf16>
int launch_fast(const void* a, const void* b, float* c, int m, int n, int k, hipStream_t stream) {
    const long long tiles = static_cast<long long>((m + kFBM - 1) / kFBM) * ((n + kFBN - 1) / kFBN);
    if (tiles > 0x7fffffffLL) return hipErrorInvalidValue;
    hipLaunchKernelGGL((matmul_mfma16_fast<kBf16>), dim3(static_cast<unsigned>(tiles)), dim3(kFThreads), 0,
                       stream, static_cast<const unsigned short*>(a), static_cast<const unsigned short*>(b), c, m, n,
                       k);
    return hipGetLastError();
}

bool aligned(const void* p, std::uintptr_t bytes) { return reinterpret_cast<std::uintptr_t>(p) % bytes == 0; }

int split_len(int k, int splits, int step) {
    if (splits <= 1) return std::max(k, 1);
    const int per = (k + splits - 1) / splits;
    return (per + step - 1) / step * step;
}

template <bool kBf16, bool kF32In>
int launch16(const void* a, const void* b, float* c, int m, int n, int k, hipStream_t stream, int splits,
             float* workspace) {
    const int k_split = split_len(k, splits, kBK);
    const int depth = std::max(1, (k + k_split - 1) / k_split);
    if (depth > 1 && workspace == nullptr) return hipErrorInvalidValue;
    const dim3 grid((n + kBN - 1) / kBN, (m + kBM - 1) / kBM, depth);
    const std::uintptr_t align = kF32In ? 16 : 8;
    const bool vec = n % 4 == 0 && k % 4 == 0 && aligned(a, align) && aligned(b, align);
    float* ws = depth > 1 ? workspace : nullptr;
    if (vec) {
        hipLaunchKernelGGL((matmul_mfma16<kBf16, kF32In, true>), grid, dim3(256), 0, stream, a, b, c, m, n, k, k_split, ws);
    } else {
        hipLaunchKernelGGL((matmul_mfma16<kBf16, kF32In, false>), grid, dim3(256), 0, stream, a, b, c, m, n, k, k_split, ws);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess || depth == 1) return e;
    return mchip_sum_split_partials(workspace, c, static_cast<std::size_t>(m) * n, depth, stream);
}

__global__ void __launch_bounds__(256) convert_kernel(const float* __restrict__ in, unsigned short* __restrict__ out,
                                                      std::size_t count, int bf16) {
    const std::size_t stride = static_cast<std::size_t>(gridDim.x) * 256;
    for (std::size_t i = static_cast<std::size_t>(blockIdx.x) * 256 + threadIdx.x; i < count; i += stride) {
        out[i] = bf16 ? to_bf16_bits(in[i]) : to_f16_bits(in[i]);
    }
}

}  // namespace

extern "C" int mchip_launch_tensor_core(int kernel, const float* a, const float* b, float* c, int m, int n, int k,
                                        void* stream, int splits, float* workspace) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (m < 1 || n < 1 || k < 1) return hipErrorInvalidValue;
    switch (kernel) {
        case kTensorCoreBf16: return launch16<true, true>(a, b, c, m, n, k, s, splits, workspace);
        case kTensorCoreF16: return launch16<false, true>(a, b, c, m, n, k, s, splits, workspace);
        case kTensorCoreTf32: return hipErrorNotSupported;
        default: return hipErrorInvalidValue;
    }
}

extern "C" int mchip_launch_matmul_lowp(int kernel, int dtype, const void* a, const void* b, float* c, int m, int n,
                                        int k, void* stream, int splits, float* workspace) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (m < 1 || n < 1 || k < 1) return hipErrorInvalidValue;
    if (kernel == kTensorCoreTf32) return hipErrorNotSupported;
    const bool fast = fast_eligible(a, b, c, m, n, k, splits);
    if (kernel == kTensorCoreBf16 && dtype == MCHIP_DTYPE_BF16) {
        return fast ? launch_fast<true>(a, b, c, m, n, k, s) : launch16<true, false>(a, b, c, m, n, k, s, splits, workspace);
    }
    if (kernel == kTensorCoreF16 && dtype == MCHIP_DTYPE_F16) {
        return fast ? launch_fast<false>(a, b, c, m, n, k, s) : launch16<false, false>(a, b, c, m, n, k, s, splits, workspace);
    }
    return hipErrorInvalidValue;
}

extern "C" int mchip_matmul_supported(int kernel) { return kernel != kTensorCoreTf32; }

extern "C" int mchip_matmul_blocks_per_cu(int kernel) {
    int blocks = 0;
    hipError_t e = hipErrorInvalidValue;
    switch (kernel) {
        case kTensorCoreBf16:
            e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, matmul_mfma16<true, true, true>, 256, 0);
            break;
        case kTensorCoreF16:
            e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, matmul_mfma16<false, true, true>, 256, 0);
            break;
        default: return 2;
    }
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return 1;
    }
    return std::max(blocks, 1);
}

extern "C" int mchip_convert_f32(int dtype, const float* in, void* out, size_t count, void* stream) {
    if (dtype != MCHIP_DTYPE_BF16 && dtype != MCHIP_DTYPE_F16) return hipErrorInvalidValue;
    const unsigned blocks = static_cast<unsigned>(std::max<std::size_t>(1, std::min<std::size_t>((count + 255) / 256, 8192)));
    hipLaunchKernelGGL(convert_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream), in,
                       static_cast<unsigned short*>(out), count, dtype == MCHIP_DTYPE_BF16 ? 1 : 0);
    return hipGetLastError();
}
