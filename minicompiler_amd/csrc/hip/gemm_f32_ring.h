// FP32 matrix-core GEMM body for gfx950 (v_mfma_f32_32x32x2_f32) with an LDS
// ring fed by direct global -> LDS loads and persistent blocks that walk
// their tiles in sequence. Shared by the ahead-of-time kernels
// (matmul_fp32.hip, identity epilogue) and the GEMMs compiled at run time
// with a fused elementwise epilogue. No standard or HIP headers, so hipRTC
// compiles it as is; it uses the split-K helpers of gemm_split_arrival.h,
// which the includer puts before it.
//
// Same arithmetic as the two-stage body in gemm_f32_mfma.h: each C element
// is accumulated by the same v_mfma_f32_32x32x2_f32 sequence (the 32-wide K
// step split into k and k + 16 slot pairs, four k per LDS read), so every
// configuration here and that body give identical bits, and any of them may
// serve a request they all accept.
//
// Requirements (checked by the host): K (and the split size) a multiple of
// 32, N a multiple of 4, A, B, C and the partials 16-byte aligned, every
// split non-empty; counters (when given): one zeroed unsigned per tile.
// Rows past M and columns past N are clamped to the last row / column
// chunk, so every load is in bounds; what they bring only reaches C elements
// that are not stored.
#pragma once

typedef float mc_ring_f32x4 __attribute__((ext_vector_type(4)));
typedef float mc_ring_f32x2 __attribute__((ext_vector_type(2)));
typedef float mc_ring_f32x16 __attribute__((ext_vector_type(16)));
#define MC_RING_LDS __attribute__((address_space(3)))

// Float vectors of 1, 2 or 4 lanes, for B reads and C stores.
template <int N>
struct McRingVec;
template <>
struct McRingVec<1> {
    typedef float type;
    static __device__ __forceinline__ float get(type v, int) { return v; }
    static __device__ __forceinline__ void set(type& v, int, float x) { v = x; }
};
template <>
struct McRingVec<2> {
    typedef mc_ring_f32x2 type;
    static __device__ __forceinline__ float get(type v, int i) { return v[i]; }
    static __device__ __forceinline__ void set(type& v, int i, float x) { v[i] = x; }
};
template <>
struct McRingVec<4> {
    typedef mc_ring_f32x4 type;
    static __device__ __forceinline__ float get(type v, int i) { return v[i]; }
    static __device__ __forceinline__ void set(type& v, int i, float x) { v[i] = x; }
};

// A configuration: block tile kBM x kBN, K step 32, kWaves waves each owning
// a kWM x kWN quadrant as (kWM / 32) x (kWN / 32) 32x32 accumulators, and a
// ring of kStages LDS stages. Lane l of a wave holds, for its accumulators'
// column blocks j < kBJ, the columns wc + kBJ (l % 32) + j: one 4-, 8- or
// 16-byte LDS read gives a lane the B values of all its column blocks, and C
// is stored kBJ floats at a time. The MFMA sequence of each C element does
// not depend on this assignment.
template <int kBM_, int kBN_, int kWM_, int kWN_, int kWaves_, int kStages_, bool kStaged_ = false>
struct McRingCfg {
    // kStaged: the fetch goes through registers (a 16-byte global load one
    // step ahead, written to LDS the next step) instead of direct loads.
    static constexpr bool kStaged = kStaged_;
    static constexpr int kBM = kBM_, kBN = kBN_, kBK = 32;
    static constexpr int kWM = kWM_, kWN = kWN_, kWaves = kWaves_, kStages = kStages_;
    static constexpr int kThreads = kWaves * 64;
    static constexpr int kWavesN = kBN / kWN;
    static constexpr int kAI = kWM / 32, kBJ = kWN / 32;
    static constexpr int kABytes = kBM * kBK * 4;
    static constexpr int kBRow = kBN * 4;  // bytes of one k row of B
    static constexpr int kStage = kABytes + kBK * kBRow;
    // 1 KiB fetch blocks per wave and step: A has kBM / 8, B kBK kBN / 256.
    static constexpr int kBBlocks = kBK * kBRow / 1024;
    static constexpr int kFA = kBM / 8 / kWaves, kFB = kBBlocks / kWaves;
    static constexpr int kFetch = kFA + kFB;
    static constexpr int kLds = kStages * kStage;
    static_assert((kBM / kWM) * kWavesN == kWaves, "waves tile the block");
    static_assert(kFA * kWaves * 8 == kBM && kFB * kWaves == kBBlocks, "fetch blocks split evenly");
    static_assert(kBN == 128 || kBN == 256, "B rows of 512 or 1024 bytes");
    static_assert(kBJ == 1 || kBJ == 2 || kBJ == 4, "column blocks per wave");
};

// The configurations the library runs (mchip_f32_ring_plan picks one by a
// cost model of the rounds each needs and its measured efficiency):
//   big:  one block of 4 waves per CU, 256x256 tiles, 128x128 per wave (16
//         accumulators, in AGPRs), 2 stages of 64 KiB, direct fetch; since
//         the staged fetch became buffer loads interleaved with the MFMAs,
//         wide is 1-4% faster on every shape both fill, and big runs only
//         when forced (ring=big);
//   wide: up to two blocks of 4 waves per CU, 128x128 tiles, 64x64 per wave
//         (accumulators in VGPRs), 2 stages, fetch staged through registers
//         a step ahead (measured 3-7% faster than its direct-fetch form, and
//         than a 4-stage direct-fetch form with one block per CU, on every
//         shape it is chosen for; with one block of 4 waves per SIMD set a
//         direct fetch instruction holds up the wave's MFMA issue);
//   wide8: the same tiles in one block of 8 waves (two per SIMD, 32x64 per
//         wave), for grids of at most one 128x128 tile (or tile-split) per
//         CU: a wave's waits overlap the other wave's MFMAs (8192x512x2048
//         131.1 against 134.0 us, 2048^3 130.9 against 134.1 us, 1024^3 in 4
//         splits 27.2 against 27.7 us on an MI355X; 256x256 tiles with 8
//         waves gained nothing);
//   thin: for M <= 32 (HBM-bound on B): 32x128 tiles, 4 waves of 32x32, 6
//         stages of 20 KiB keeping more of B in flight, so a 128-row tile's
//         MFMA work on clamped rows no longer dominates;
//   mid:  64x128 tiles, 4 waves of 32x64, 3 stages of 24 KiB, up to two
//         blocks per CU. Chosen only by the autotuner (with thin at any M):
//         small products split K less with smaller tiles (1024 x 2048 x 512
//         unsplit on mid: 23.8 us against 31.4 us for wide with 2 splits).
using McRingBig = McRingCfg<256, 256, 128, 128, 4, 2>;
using McRingWide = McRingCfg<128, 128, 64, 64, 4, 2, true>;
using McRingWide8 = McRingCfg<128, 128, 32, 64, 8, 2, true>;
using McRingThin = McRingCfg<32, 128, 32, 32, 4, 6>;
using McRingMid = McRingCfg<64, 128, 32, 64, 4, 3>;

// LDS layout of a stage (bytes):
//   A at 0: kBM / 8 blocks of 1 KiB, block rb holding rows 8 rb .. 8 rb + 7
//     of the tile. Chunk c (k 4c .. 4c + 3, 16 bytes) of row r sits at
//     position p = 16 (c / 2) + 8 ((c % 2) ^ (rb % 2)) + r % 8 of its block.
//     An A-fragment read (32 lanes: 32 consecutive rows, one chunk) then
//     puts every 16 lanes on 16 distinct 16-byte bank groups; a fetch
//     instruction (lane l -> position l) still covers 8 whole 128-byte rows.
//   B after A: k row kk at kBRow kk, n-contiguous, its 16-byte chunk g
//     stored at g ^ 8 (kk / 16 % 2). The two half-waves of a read take k rows
//     kk and kk + 16 and the same columns: with 4-byte reads the XOR puts
//     them on disjoint banks; 8- and 16-byte reads stay contiguous within
//     each half-wave (the XOR permutes within 256-byte windows).

__device__ __forceinline__ int mc_ring_min(int a, int b) { return a < b ? a : b; }

// Where this lane's fetches of one step come from, for one unit (a tile, or
// a tile's share of K under split-K): buffer resources based at the unit's
// origin in A (row row0, column kb) and in B (row kb, column col0), the
// lane's byte offset from each origin for its chunks of step 0, and the
// bytes between consecutive K steps (kBK * 4 in A, kBK rows in B), which go
// in the scalar offset. A buffer load takes its per-lane address as a
// 32-bit offset added to a base held in scalar registers, so no vector
// instruction computes addresses in the main loop (the 64-bit global
// addresses it replaces took one VALU add per load; 8192x512x2048 ran 4%
// slower so). The host guarantees that every offset fits in 31 bits
// (mchip_ring_offsets_fit).
template <class Cfg>
struct McRingFetch {
    __amdgpu_buffer_rsrc_t a_rsrc, b_rsrc;
    int a_off[Cfg::kFA];
    int b_off[Cfg::kFB];
    int b_step;
};

struct McRingUnit {
    int row0, col0, kb, steps, split;
};

// A stage parity as a type, for the staged main loop's steps.
template <int V>
struct McRingParity {
    static constexpr int value = V;
};

// Raw buffer resource over `base` (stride 0: byte-addressed; the offsets
// stay inside the operand, so the range is not what bounds them).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t mc_ring_rsrc(const float* base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), 0, 0x7fffffff, 0x00020000);
}

// Non-temporal buffer stores of 1, 2 or 4 floats at byte offset voffset +
// soffset from the resource's base (plain functions, like the LDS load).
__device__ __forceinline__ void mc_ring_buffer_store(float v, __amdgpu_buffer_rsrc_t r, int voffset, int soffset) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), r, voffset, soffset, 2);
}
typedef unsigned mc_ring_u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned mc_ring_u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void mc_ring_buffer_store(mc_ring_f32x2 v, __amdgpu_buffer_rsrc_t r, int voffset, int soffset) {
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(mc_ring_u32x2, v), r, voffset, soffset, 2);
}
__device__ __forceinline__ void mc_ring_buffer_store(mc_ring_f32x4 v, __amdgpu_buffer_rsrc_t r, int voffset, int soffset) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(mc_ring_u32x4, v), r, voffset, soffset, 2);
}

// Global -> LDS without registers: buffer_load_dwordx4 ... lds writes lane
// l's 16 bytes at (LDS base + 16 l). (A plain function: called in a
// template, the builtin failed the host pass of the AOT build.)
__device__ __forceinline__ void mc_ring_buffer_to_lds(__amdgpu_buffer_rsrc_t rsrc, MC_RING_LDS unsigned char* dst,
                                                      int voffset, int soffset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, reinterpret_cast<MC_RING_LDS void*>(dst), 16, voffset, soffset, 0, 0);
}

// Instruction idx of a step's direct fetch: A blocks first, then B blocks.
template <class Cfg>
__device__ __forceinline__ void mc_ring_fetch_one(MC_RING_LDS unsigned char* wr, const McRingFetch<Cfg>& f, int wave,
                                                  int t, int idx) {
    if (idx < Cfg::kFA) {
        mc_ring_buffer_to_lds(f.a_rsrc, wr + (wave * Cfg::kFA + idx) * 1024, f.a_off[idx], t * (Cfg::kBK * 4));
    } else {
        const int i = idx - Cfg::kFA;
        mc_ring_buffer_to_lds(f.b_rsrc, wr + Cfg::kABytes + (wave * Cfg::kFB + i) * 1024, f.b_off[i], t * f.b_step);
    }
}

// The staged fetch: instruction idx of a step as a 16-byte buffer load into
// registers, and later the store of those registers to the LDS position the
// direct load would fill (so both fetch forms give the same stage contents).
template <class Cfg>
__device__ __forceinline__ mc_ring_f32x4 mc_ring_load_one(const McRingFetch<Cfg>& f, int t, int idx) {
    if (idx < Cfg::kFA)
        return __builtin_bit_cast(mc_ring_f32x4,
                                  __builtin_amdgcn_raw_buffer_load_b128(f.a_rsrc, f.a_off[idx], t * (Cfg::kBK * 4), 0));
    return __builtin_bit_cast(mc_ring_f32x4,
                              __builtin_amdgcn_raw_buffer_load_b128(f.b_rsrc, f.b_off[idx - Cfg::kFA], t * f.b_step, 0));
}

template <class Cfg>
__device__ __forceinline__ void mc_ring_store_one(MC_RING_LDS unsigned char* wr, int wave, int lane, int idx,
                                                  mc_ring_f32x4 v) {
    const int blk = idx < Cfg::kFA ? (wave * Cfg::kFA + idx) * 1024
                                   : Cfg::kABytes + (wave * Cfg::kFB + idx - Cfg::kFA) * 1024;
    *reinterpret_cast<MC_RING_LDS mc_ring_f32x4*>(wr + blk + 16 * lane) = v;
}

// All of a step's fetch instructions (the prologue's): direct loads, or for
// the staged configurations the loads into registers and their LDS stores
// (so a staged kernel issues no direct load at all, and the compiler's
// count of loads in flight at the main loop stays exact: with a direct load
// possibly in flight it waited for every load before each LDS store).
template <class Cfg>
__device__ __forceinline__ void mc_ring_fetch(MC_RING_LDS unsigned char* wr, const McRingFetch<Cfg>& f, int wave,
                                              int t) {
    if constexpr (Cfg::kStaged) {
        const int lane = static_cast<int>(threadIdx.x) & 63;
        mc_ring_f32x4 v[Cfg::kFetch];
#pragma unroll
        for (int idx = 0; idx < Cfg::kFetch; ++idx) v[idx] = mc_ring_load_one<Cfg>(f, t, idx);
#pragma unroll
        for (int idx = 0; idx < Cfg::kFetch; ++idx) mc_ring_store_one<Cfg>(wr, wave, lane, idx, v[idx]);
    } else {
#pragma unroll
        for (int idx = 0; idx < Cfg::kFetch; ++idx) mc_ring_fetch_one<Cfg>(wr, f, wave, t, idx);
    }
}

// One step: multiply the step held in `rd` (the MFMA sequence of the
// two-stage body) and, with do_fetch, fetch a later step into `wr`, its
// instructions spread over the first 8 of the step's 16 MFMA groups. Issued
// all at once, they stalled the wave in the memory pipe (each instruction
// moves 1 KiB, and the CU's pipe takes a few tens of cycles per
// instruction) while its matrix unit idled; spread, the pipe keeps up and
// every fetch still has half a step to land. `rd` and `wr` are distinct
// stages; declaring them __restrict__ gives the LDS reads alias scopes that
// keep the compiler from making them wait for the fetch.
//
// The 16 groups (q, e) of a step each take one B read (and, at e = 0, the
// K group's A reads). The reads of group t + 1 are issued with the MFMAs of
// group t, into the other of two register sets: the MFMAs of group t then
// cover the LDS latency of group t + 1 (left to itself the compiler reuses
// one register set and waits for each read right before its MFMAs). Within
// a group the memory instructions are interleaved with the MFMAs, one of
// each kind (LDS write, load, LDS read) after each MFMA, so each issues while
// an MFMA runs: issued as one block between two groups' MFMAs, they left the
// matrix unit idle while the wave issued them (8192x512x2048 on the wide
// configuration: 126.2 us so, 122.9 us interleaved, one MI355X).
//
// Staged configurations: the registers loaded one step ago are written to
// `wr`, and the next fetch is loaded into the same registers right behind
// each write, so every load has a whole step to land. Both happen at every
// step (past the last step they move data no step reads, into a stage no
// later step reads): with either one conditional, the compiler's wait before
// each write would also wait for this step's loads.
template <class Cfg>
__device__ __forceinline__ void mc_ring_step(const MC_RING_LDS unsigned char* __restrict__ rd,
                                             MC_RING_LDS unsigned char* __restrict__ wr, bool do_fetch,
                                             const McRingFetch<Cfg>& f, int wave, int fetch_t,
                                             const int (&a_off)[Cfg::kAI][4], int b_off,
                                             mc_ring_f32x16 (&acc)[Cfg::kAI][Cfg::kBJ],
                                             mc_ring_f32x4 (&staged)[Cfg::kFetch]) {
    typedef McRingVec<Cfg::kBJ> BV;
    typedef typename BV::type BT;
    mc_ring_f32x4 av[2][Cfg::kAI];
    BT bv[2];
#pragma unroll
    for (int i = 0; i < Cfg::kAI; ++i) av[0][i] = *reinterpret_cast<const MC_RING_LDS mc_ring_f32x4*>(rd + a_off[i][0]);
    bv[0] = *reinterpret_cast<const MC_RING_LDS BT*>(rd + b_off);
#pragma unroll
    for (int t = 0; t < 16; ++t) {
        const int q = t >> 2, e = t & 3;
        if constexpr (Cfg::kStaged) {
            const int lane = static_cast<int>(threadIdx.x) & 63;
#pragma unroll
            for (int idx = 0; idx < Cfg::kFetch; ++idx) {
                if (idx * 8 / Cfg::kFetch == t) {
                    mc_ring_store_one<Cfg>(wr, wave, lane, idx, staged[idx]);
                    staged[idx] = mc_ring_load_one<Cfg>(f, fetch_t, idx);
                }
            }
        } else if (do_fetch) {
#pragma unroll
            for (int idx = 0; idx < Cfg::kFetch; ++idx) {
                if (idx * 8 / Cfg::kFetch == t) mc_ring_fetch_one<Cfg>(wr, f, wave, fetch_t, idx);
            }
        }
        if (t + 1 < 16) {
            if (((t + 1) & 3) == 0) {
#pragma unroll
                for (int i = 0; i < Cfg::kAI; ++i)
                    av[(q + 1) & 1][i] = *reinterpret_cast<const MC_RING_LDS mc_ring_f32x4*>(rd + a_off[i][q + 1]);
            }
            bv[(t + 1) & 1] = *reinterpret_cast<const MC_RING_LDS BT*>(rd + b_off + (t + 1) * Cfg::kBRow);
        }
#pragma unroll
        for (int i = 0; i < Cfg::kAI; ++i)
#pragma unroll
            for (int j = 0; j < Cfg::kBJ; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[q & 1][i][e], BV::get(bv[t & 1], j), acc[i][j], 0,
                                                                 0, 0);
#pragma unroll
        for (int r = 0; r < Cfg::kAI * Cfg::kBJ; ++r) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // an MFMA
            __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // an LDS write
            __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // a load
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // an LDS read
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

// s_waitcnt vmcnt(v) lgkmcnt(0), expcnt not waited on (gfx9 encoding).
#define MC_RING_WAIT(v) __builtin_amdgcn_s_waitcnt(0x0070 | ((v) & 15) | (((v) >> 4) << 14))

// Wait until at most `later` fetch groups of kFetch instructions are in
// flight (later <= kMax, the ring's stages minus two), and for LDS reads.
template <int kFetch, int kMax>
__device__ __forceinline__ void mc_ring_wait_later(int later) {
    if constexpr (kMax > 0) {
        if (later >= kMax) {
            MC_RING_WAIT(kMax * kFetch);
            return;
        }
        mc_ring_wait_later<kFetch, kMax - 1>(later);
    } else {
        MC_RING_WAIT(0);
    }
}

// A workgroup barrier without a memory fence; the compiler may not move
// memory operations or MFMAs across it.
__device__ __forceinline__ void mc_ring_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

// The store of one unit's accumulators: acc[i][j] value v of lane l is row
// row0 + 32 i + 8 (v / 4) + v % 4 (row0 includes the lane's 4 (l / 32)),
// column col + j. The kBJ columns of a lane are stored together: with N a
// multiple of 4 they are all inside C or all past its edge (the caller skips
// the latter). kCheck: some rows may be past M. Without it the store is
// straight-line code.
// With one or two columns per lane (every configuration but big) the
// epilogue runs over a batch of rows (32 or 64 values) before the batch's
// first store: with each row stored right after its epilogue, the compiler
// waited for the epilogue's operand loads a few rows at a time (9 waits per
// tile of the MLP's GEMM2); batched, a row's two residual floats merge into
// one 8-byte load and the batch's loads are in flight before one wait (2
// waits per tile). The MLP's GEMM2 with b2 + residual (wide): 139.2-139.6 us
// against 140.8-141.1. Big keeps each row's store right after its epilogue
// (its 4 columns per lane already load a bias once): batched, its GEMM with
// bias + GELU took 136.5-136.7 us against 135.3 (one MI355X, 3 runs each).
// C goes out with non-temporal stores (every CU stores its tiles at about
// the same moment at the end of a one-tile-per-CU launch): same bits, the
// MLP's GEMM2 with b2 + residual 138.4-138.6 us against 139.4-139.6 and
// 2048^3 131.0 against 132.1 us on one MI355X; the MLP's step and the other
// sweep rows within 0.2%.
// kSplit: raw partial sums that this launch adds, stored float by float
// with device-scope stores (mc_split_store).
template <class Cfg, bool kCheck, typename Epilogue, bool kSplit = false>
__device__ __forceinline__ void mc_ring_store(const mc_ring_f32x16 (&acc)[Cfg::kAI][Cfg::kBJ], float* __restrict__ out,
                                              int tile_row0, int tile_col0, int row0, int col, int m, int n, bool raw,
                                              const Epilogue& epilogue) {
    typedef McRingVec<Cfg::kBJ> BV;
    auto row_of = [&](int i, int v) { return row0 + 32 * i + 8 * (v >> 2) + (v & 3); };
    // Buffer stores from the tile's origin in C: the lane's byte offset in a
    // vector register, each row's distance from the lane's first row (a
    // multiple of 4 n) in a scalar one, so no vector instruction computes a
    // store address (the 64-bit addresses they replace took about four
    // vector ALU instructions per store, which a SIMD does not run beside
    // MFMAs). The host keeps the offsets below 2^31 (256 rows of C).
    const __amdgpu_buffer_rsrc_t c_rsrc = mc_ring_rsrc(out + static_cast<long long>(tile_row0) * n + tile_col0);
    const int c_off = 4 * ((row0 - tile_row0) * n + (col - tile_col0));
    auto row_step = [&](int i, int v) { return 4 * n * (32 * i + 8 * (v >> 2) + (v & 3)); };
    if constexpr (kSplit) {
#pragma unroll
        for (int i = 0; i < Cfg::kAI; ++i)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int row = row_of(i, v);
                if (kCheck && row >= m) continue;
                const long long at = static_cast<long long>(row) * n + col;
#pragma unroll
                for (int j = 0; j < Cfg::kBJ; ++j) mc_split_store(out + at + j, acc[i][j][v]);
            }
        return;
    }
    if constexpr (Cfg::kBJ > 2) {
#pragma unroll
        for (int i = 0; i < Cfg::kAI; ++i)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int row = row_of(i, v);
                if (kCheck && row >= m) continue;
                const long long at = static_cast<long long>(row) * n + col;
                typename BV::type o;
#pragma unroll
                for (int j = 0; j < Cfg::kBJ; ++j) {
                    const float x = acc[i][j][v];
                    BV::set(o, j, raw ? x : epilogue(x, static_cast<unsigned>(at + j)));
                }
                mc_ring_buffer_store(o, c_rsrc, c_off, row_step(i, v));
            }
        return;
    }
    constexpr int kRowsPerBatch = Cfg::kAI % 2 == 0 ? 2 : 1;
#pragma unroll
    for (int i0 = 0; i0 < Cfg::kAI; i0 += kRowsPerBatch) {
        typename BV::type o[kRowsPerBatch][16];
#pragma unroll
        for (int di = 0; di < kRowsPerBatch; ++di)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int row = row_of(i0 + di, v);
                // A row past M reads no epilogue operand (nor is it stored).
                if (kCheck && row >= m) {
                    o[di][v] = typename BV::type{};
                    continue;
                }
                // The epilogue's element index, computed in the 32 bits it
                // takes (the same value as the 64-bit offset truncated).
                const unsigned at = static_cast<unsigned>(row) * static_cast<unsigned>(n) + static_cast<unsigned>(col);
#pragma unroll
                for (int j = 0; j < Cfg::kBJ; ++j) {
                    const float x = acc[i0 + di][j][v];
                    BV::set(o[di][v], j, raw ? x : epilogue(x, at + j));
                }
            }
#pragma unroll
        for (int di = 0; di < kRowsPerBatch; ++di)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int row = row_of(i0 + di, v);
                if (kCheck && row >= m) continue;
                mc_ring_buffer_store(o[di][v], c_rsrc, c_off, row_step(i0 + di, v));
            }
    }
}

// C tile (row0, col0) from the partials of its `splits` K splits, added in
// split order (a lane issues its loads of 8 splits before it adds them) and
// stored through the epilogue, 16 bytes per lane and step.
template <class Cfg, typename Epilogue>
__device__ __forceinline__ void mc_ring_fold(const float* __restrict__ partial, float* __restrict__ c, int row0,
                                             int col0, int m, int n, int splits, const Epilogue& epilogue) {
    constexpr int kQ = Cfg::kBN / 4, kChunk = 8;
    const long long plane = static_cast<long long>(m) * n;
    for (int t = threadIdx.x; t < Cfg::kBM * kQ; t += Cfg::kThreads) {
        const int row = row0 + t / kQ, col = col0 + 4 * (t % kQ);
        if (row >= m || col >= n) continue;
        const long long at = static_cast<long long>(row) * n + col;
        auto load = [&](int z) {
            const float* p = partial + z * plane + at;
            return mc_ring_f32x4{mc_split_load(p), mc_split_load(p + 1), mc_split_load(p + 2), mc_split_load(p + 3)};
        };
        mc_ring_f32x4 sum = load(0);
        for (int z0 = 1; z0 < splits; z0 += kChunk) {
            mc_ring_f32x4 x[kChunk];
#pragma unroll
            for (int i = 0; i < kChunk; ++i) x[i] = load(z0 + i < splits ? z0 + i : splits - 1);
#pragma unroll
            for (int i = 0; i < kChunk; ++i)
                if (z0 + i < splits) sum += x[i];
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) sum[j] = epilogue(sum[j], static_cast<unsigned>(at + j));
        *reinterpret_cast<mc_ring_f32x4*>(c + at) = sum;
    }
}

// The C tiles (and K splits) of an M x N x K product, `splits` splits of
// `k_split` each: unit u is split u / tiles of tile u % tiles (tiles in
// row-major order). Blocks are persistent: with the grid a multiple of 8,
// block b runs on XCD b % 8 and takes the units of that XCD's contiguous
// eighth of the list, so the blocks sharing an XCD's L2 share A row bands
// and B column panels; otherwise block b takes units b, b + grid, ...
// With one split the epilogue maps each accumulated value v of element
// i = row n + col to what is stored; with several, the raw partial sums go
// to `partial` (split s at s m n) and the epilogue is applied where the
// splits are summed: in this launch, by the last block to finish a split of
// the tile, when `counters` is given (not null), else by a separate launch.
template <class Cfg, typename Epilogue>
__device__ __forceinline__ void mc_gemm_f32_ring(const float* __restrict__ a, const float* __restrict__ b,
                                                 float* __restrict__ c, int m, int n, int k, int k_split, int splits,
                                                 float* __restrict__ partial, unsigned* __restrict__ counters,
                                                 const Epilogue& epilogue) {
    typedef McRingVec<Cfg::kBJ> BV;
    __shared__ __attribute__((aligned(1024))) unsigned char smem[Cfg::kLds];
    MC_RING_LDS unsigned char* lds = (MC_RING_LDS unsigned char*)(smem);  // generic -> LDS address space

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int tiles_n = (n + Cfg::kBN - 1) / Cfg::kBN;
    const int tiles = ((m + Cfg::kBM - 1) / Cfg::kBM) * tiles_n;
    const int units = tiles * splits;

    // This block's units: first, first + stride, ... (count of them).
    const int grid = static_cast<int>(gridDim.x);
    int first, stride, count;
    if (grid % 8 == 0) {
        const int x = static_cast<int>(blockIdx.x) % 8, j = static_cast<int>(blockIdx.x) / 8;
        const int lo = static_cast<int>(static_cast<long long>(x) * units / 8);
        const int hi = static_cast<int>(static_cast<long long>(x + 1) * units / 8);
        first = lo + j;
        stride = grid / 8;
        count = first < hi ? (hi - first + stride - 1) / stride : 0;
    } else {
        first = static_cast<int>(blockIdx.x);
        stride = grid;
        count = first < units ? (units - first + stride - 1) / stride : 0;
    }
    auto unit_of = [&](int i) {
        const int u = first + i * stride;
        McRingUnit r;
        r.split = u / tiles;
        const int t = u % tiles;
        r.row0 = (t / tiles_n) * Cfg::kBM;
        r.col0 = (t % tiles_n) * Cfg::kBN;
        r.kb = r.split * k_split;
        const int ke = mc_ring_min(k, r.kb + k_split);
        r.steps = (ke - r.kb) / Cfg::kBK;
        return r;
    };
    // A: wave w fills blocks rb = kFA w + i; lane l -> row 8 rb + l % 8,
    // chunk 2 (l / 16) + ((l / 8 % 2) ^ (rb % 2)). B: wave w fills blocks
    // bb = kFB w + i, each 1024 / kBRow k rows; lane l -> k row
    // bb 1024 / kBRow + l / (kBRow / 16), physical chunk l % (kBRow / 16),
    // logical chunk that ^ 8 (k row / 16 % 2).
    constexpr int kLanesPerBRow = Cfg::kBRow / 16;
    // Offsets are from the unit's origin; clamped rows and columns are at or
    // past it (row0 <= m - 1, col0 <= n - 4).
    auto fetch_of = [&](const McRingUnit& u) {
        McRingFetch<Cfg> f;
        f.a_rsrc = mc_ring_rsrc(a + static_cast<long long>(u.row0) * k + u.kb);
        f.b_rsrc = mc_ring_rsrc(b + static_cast<long long>(u.kb) * n + u.col0);
#pragma unroll
        for (int i = 0; i < Cfg::kFA; ++i) {
            const int rb = Cfg::kFA * wave + i;
            const int r = mc_ring_min(u.row0 + rb * 8 + (lane & 7), m - 1);
            const int ch = 2 * (lane >> 4) + (((lane >> 3) & 1) ^ (rb & 1));
            f.a_off[i] = 4 * ((r - u.row0) * k + 4 * ch);
        }
#pragma unroll
        for (int i = 0; i < Cfg::kFB; ++i) {
            const int kk = (Cfg::kFB * wave + i) * (1024 / Cfg::kBRow) + lane / kLanesPerBRow;
            const int g = (lane % kLanesPerBRow) ^ (8 * ((kk >> 4) & 1));
            const int col = mc_ring_min(u.col0 + 4 * g, n - 4);
            f.b_off[i] = 4 * (kk * n + col - u.col0);
        }
        f.b_step = 4 * Cfg::kBK * n;
        return f;
    };

    // Read offsets. Wave (wm, wn) owns rows kWM wm .. and columns kWN wn ..;
    // lane l reads A rows wr + 32 i + l % 32 and B columns
    // wc + kBJ (l % 32) .. + kBJ - 1, k slot l / 32.
    const int wr = (wave / Cfg::kWavesN) * Cfg::kWM, wc = (wave % Cfg::kWavesN) * Cfg::kWN;
    const int half = lane >> 5, li = lane & 31;
    int a_off[Cfg::kAI][4];
#pragma unroll
    for (int i = 0; i < Cfg::kAI; ++i) {
        const int row = wr + 32 * i + li;
        const int rb = row >> 3;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int ch = 4 * half + q;
            a_off[i][q] = rb * 1024 + 16 * (16 * (ch >> 1) + 8 * ((ch & 1) ^ (rb & 1)) + (row & 7));
        }
    }
    const int lcol = wc + Cfg::kBJ * li;  // first of this lane's columns in the tile
    const int b_off = Cfg::kABytes + half * 16 * Cfg::kBRow + (((lcol >> 2) ^ (8 * half)) << 4) + (lcol & 3) * 4;

    // Total steps of this block, and the fetch cursor (unit fi, step ft).
    int total = 0;
    for (int i = 0; i < count; ++i) total += unit_of(i).steps;
    int fi = 0, ft = 0;
    McRingUnit fu = unit_of(0);
    McRingFetch<Cfg> fetch = fetch_of(fu);
    auto advance = [&]() {
        if (++ft == fu.steps) {
            ft = 0;
            if (++fi < count) {
                fu = unit_of(fi);
                fetch = fetch_of(fu);
            }
        }
    };

    // Stage of the next fetch and of the next step to multiply.
    int ws = 0, rs = 0;
    auto next = [](int s) { return s + 1 == Cfg::kStages ? 0 : s + 1; };
    int issued = 0;
    const int pre = mc_ring_min(total, Cfg::kStages - 1);
    for (; issued < pre; ++issued) {
        mc_ring_fetch<Cfg>(lds + ws * Cfg::kStage, fetch, wave, ft);
        ws = next(ws);
        advance();
    }
    // Staged: the registers hold the fetch of step `pre` (loaded, not yet
    // written). Past the block's last unit the cursor wraps to the start of
    // that unit, so every load stays in bounds.
    mc_ring_f32x4 staged[Cfg::kFetch];
    if constexpr (Cfg::kStaged) {
        if (total > 0) {
#pragma unroll
            for (int idx = 0; idx < Cfg::kFetch; ++idx) staged[idx] = mc_ring_load_one<Cfg>(fetch, ft, idx);
            advance();
        }
    }

    int g = 0;  // steps consumed
    for (int ui = 0; ui < count; ++ui) {
        const McRingUnit u = unit_of(ui);
        mc_ring_f32x16 acc[Cfg::kAI][Cfg::kBJ];
#pragma unroll
        for (int i = 0; i < Cfg::kAI; ++i)
#pragma unroll
            for (int j = 0; j < Cfg::kBJ; ++j) acc[i][j] = mc_ring_f32x16{};
        if constexpr (Cfg::kStaged && Cfg::kStages == 2) {
            // Staged, two stages: step g reads stage g % 2 and writes the
            // staged registers to the other. The steps run in pairs of
            // constant parity, so each stage's LDS offsets are immediates of
            // the LDS instructions: with the stage a run-time value every
            // step spent 9 vector ALU instructions on LDS addresses, and on
            // gfx950 a SIMD does not run those beside its MFMAs. On an
            // MI355X, with the constant parities: 8192x512x2048 + b2 +
            // residual 129.7 -> 127.1 us, 4096^3 146.3 -> 148.1 TFLOP/s,
            // 8192^3 146.9 -> 149.8.
            auto step = [&](auto parity) {
                constexpr int kP = decltype(parity)::value;
                // Step g was written to LDS from registers by the prologue or
                // during step g - 1: wait for this wave's LDS writes (and
                // reads). Then every wave's writes of step g are done, and
                // every wave is done with step g - 1, whose stage this step
                // writes.
                MC_RING_WAIT(63);
                mc_ring_barrier();
                mc_ring_step<Cfg>(lds + kP * Cfg::kStage, lds + (1 - kP) * Cfg::kStage, true, fetch, wave, ft, a_off,
                                  b_off, acc, staged);
                advance();
            };
            int t = 0;
            if ((g & 1) != 0 && t < u.steps) {
                step(McRingParity<1>{});
                ++t;
                ++g;
            }
            for (; t + 1 < u.steps; t += 2, g += 2) {
                step(McRingParity<0>{});
                step(McRingParity<1>{});
            }
            if (t < u.steps) {
                step(McRingParity<0>{});
                ++t;
                ++g;
            }
        } else {
            for (int t = 0; t < u.steps; ++t, ++g) {
                if constexpr (Cfg::kStaged) {
                    // Step g was written to LDS from registers by the prologue
                    // or during step g - 1: wait for this wave's LDS writes
                    // (and reads).
                    MC_RING_WAIT(63);
                } else {
                    // Fetch groups issued after the one of step g (stores
                    // issued after it only make the wait longer): wait for
                    // that one and for this wave's LDS reads of the previous
                    // step.
                    mc_ring_wait_later<Cfg::kFetch, Cfg::kStages - 2>(issued - g - 1);
                }
                // Every wave's fetch of step g has landed, and every wave is
                // done with step g - 1, whose stage the next fetch overwrites.
                mc_ring_barrier();
                const bool more = Cfg::kStaged || issued < total;
                mc_ring_step<Cfg>(lds + rs * Cfg::kStage, lds + ws * Cfg::kStage, more, fetch, wave, ft, a_off, b_off,
                                  acc, staged);
                rs = next(rs);
                if (more) {
                    ++issued;
                    ws = next(ws);
                    advance();
                }
            }
        }
        const int col = u.col0 + lcol;
        const bool fold = splits > 1 && counters != nullptr;
        if (col < n) {
            float* __restrict__ out = splits > 1 ? partial + static_cast<long long>(u.split) * m * n : c;
            const int r0 = u.row0 + wr + 4 * half;
            if (fold) {
                if (u.row0 + Cfg::kBM <= m)
                    mc_ring_store<Cfg, false, Epilogue, true>(acc, out, u.row0, u.col0, r0, col, m, n, true, epilogue);
                else
                    mc_ring_store<Cfg, true, Epilogue, true>(acc, out, u.row0, u.col0, r0, col, m, n, true, epilogue);
            } else if (u.row0 + Cfg::kBM <= m) {
                mc_ring_store<Cfg, false>(acc, out, u.row0, u.col0, r0, col, m, n, splits > 1, epilogue);
            } else {
                mc_ring_store<Cfg, true>(acc, out, u.row0, u.col0, r0, col, m, n, splits > 1, epilogue);
            }
        }
        if (fold) {
            __shared__ int last_flag;
            const int tile = (u.row0 / Cfg::kBM) * tiles_n + u.col0 / Cfg::kBN;
            if (mc_split_last_arrival(counters + tile, splits, &last_flag))
                mc_ring_fold<Cfg>(partial, c, u.row0, u.col0, m, n, splits, epilogue);
        }
    }
    MC_RING_WAIT(0);
}
