// bf16 / fp16 matrix-core GEMM body for gfx950 on 16-bit inputs already in
// HBM, shared by the ahead-of-time kernels (matmul_mfma16.hip, identity
// epilogue) and the GEMMs compiled at run time with a fused elementwise
// epilogue (the executable's generated source embeds this file).
// Self-contained: no standard or HIP headers, so hipRTC compiles it as is.
#pragma once

typedef float mc_f32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned short mc_u16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 mc_bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 mc_f16x8_t __attribute__((ext_vector_type(8)));

template <bool kBf16>
__device__ __forceinline__ mc_f32x4_t mc_mfma16(mc_u16x8_t a, mc_u16x8_t b, mc_f32x4_t c) {
    if constexpr (kBf16) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(mc_bf16x8_t, a),
                                                       __builtin_bit_cast(mc_bf16x8_t, b), c, 0, 0, 0);
    } else {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(mc_f16x8_t, a),
                                                      __builtin_bit_cast(mc_f16x8_t, b), c, 0, 0, 0);
    }
}

// The identity epilogue: C[i] = the accumulated dot product.
struct McGemm16Store {
    __device__ __forceinline__ float operator()(float v, unsigned) const { return v; }
};

// 16-bit inputs already in HBM, K a multiple of 64, N a multiple of 8, rows
// 16-byte aligned. Block tile 256x256, 512 lanes = 8 waves in a 2x4 grid
// (two waves per SIMD), each wave a 128x64 quadrant as 8x4 accumulators of
// v_mfma_f32_16x16x32 (128 fp32 per lane, in AGPRs). One block per CU; the
// two waves of a SIMD hide each other's LDS and barrier waits.
//
// K is walked in steps of 32 through a ring of four 32 KiB LDS stages, with
// the two waves of each SIMD in ping-pong: waves 0-3 and waves 4-7 run the
// same sequence one phase apart, alternating a memory phase (issue the
// global -> LDS fetch of A for step t+3, read step t's operands from LDS into
// registers) and a compute phase (step t's 32 MFMAs, with the fetch of B for
// step t+3 issued after the first 16), so each SIMD's matrix unit is fed by
// one wave while the other loads. Phases are separated by a
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

// Packed A (the kPackedA form; mc_pack_a16 and the compiled graphs' rounding
// of fp32 operands write it): A cut into bands of 256 rows (the last band
// padded with zero rows) and each band into K steps of 32, every (band, step)
// block 16 KiB in the order of a stage's A region, so that each fetch
// instruction reads 1 KiB linearly instead of 64 bytes from each of 16 rows.
// Element (row, kk) of an M x K matrix sits at index
//   (row / 256) 256 K + (kk / 32) 8192 + (row % 256 / 16) 512 + (kk % 32 / 8) 128 + (row % 16) 8 + kk % 8.
// On an MI355X the 8192^3 bf16 product took 787-795 us so against 840-845 us
// with row-major A (timing copies, one process); the same layout for B
// gained nothing (B's fetch already reads 512 bytes per k row).

__device__ __forceinline__ int mc_min16(int a, int b) { return a < b ? a : b; }
#define MC_LDS __attribute__((address_space(3)))

constexpr int kFBM = 256, kFBN = 256, kFBK = 32;
constexpr int kFThreads = 512;
constexpr int kFWaves = kFThreads / 64;
constexpr int kFStages = 4;
constexpr int kFStage = 32 * 1024;
constexpr int kFBOffset = 16 * 1024;
constexpr int kFColFrags = 4;  // 16-column B fragments per wave (64 columns)

__device__ __forceinline__ int swz_b(int kr) { return (kr & 3) | (((kr >> 3) & 3) << 2); }

// A block tile of kRows x 256 (kRows = 256, or 128 for the halves of the
// last tiles): wave (wm, wn) of the 2x4 grid owns kRows / 2 rows as
// kRows / 32 A fragments of 16 rows. A stage holds kRows A rows (kRows / 128
// global_load_lds instructions per wave and step) and 32 k rows of B (2 per
// wave).
template <int kRows>
struct FastShape {
    static constexpr int kRowFrags = kRows / 32;
    static constexpr int kFetchA = kRows / 128;
    static constexpr int kFetch = kFetchA + 2;
};

// Per-lane addressing, set up once per block. The fetches are buffer loads
// from bases at the tile's origin in A (row row0) and B (column col0): the
// lane's 32-bit byte offset for k step 0 in a vector register, the step's
// offset (2 k0 bytes in A, 2 k0 n in B) in a scalar one, so the memory phase
// computes no addresses (the 64-bit global addresses it replaces took vector
// adds and a multiply per step). The host keeps every offset below 2^31.
template <int kRows>
struct FastLane {
    __amdgpu_buffer_rsrc_t a_rsrc, b_rsrc;
    int a_src[FastShape<kRows>::kFetchA];  // byte offset of the A chunk this lane fetches per instruction (k 0)
    int a_step;                            // bytes between consecutive K steps of A (64 row-major, 16 KiB packed)
    int b_src[2];                          // byte offset of the B chunk (k row 0)
    int b_step;                            // bytes between consecutive K steps of B
    int a_off[FastShape<kRows>::kRowFrags];  // LDS byte offsets of the A fragments
    int b_off[2][kFColFrags];                // LDS byte offsets of the two transposed B reads
    int wave;
};

// One 16-byte-per-lane buffer load into LDS (lane l at dst + 16 l). A plain
// function: called in a template, the builtin failed the host pass of the
// ahead-of-time build.
__device__ __forceinline__ void fast_buffer_to_lds(__amdgpu_buffer_rsrc_t rsrc, MC_LDS unsigned char* dst, int voffset,
                                                   int soffset) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, reinterpret_cast<MC_LDS void*>(dst), 16, voffset, soffset, 0, 0);
}

// The fetch of K step `fetch_k` into stage `wr`: this wave's kFetchA A
// instructions and its 2 B instructions.
template <int kRows>
__device__ __forceinline__ void fast_fetch_a(MC_LDS unsigned char* wr, const FastLane<kRows>& L, int fetch_k) {
    constexpr int kFA = FastShape<kRows>::kFetchA;
    MC_LDS unsigned char* sa = wr + L.wave * kFA * 1024;
#pragma unroll
    for (int i = 0; i < kFA; ++i) fast_buffer_to_lds(L.a_rsrc, sa + i * 1024, L.a_src[i], (fetch_k / kFBK) * L.a_step);
}

template <int kRows>
__device__ __forceinline__ void fast_fetch_b(MC_LDS unsigned char* wr, const FastLane<kRows>& L, int fetch_k) {
    MC_LDS unsigned char* sb = wr + kFBOffset + L.wave * 4 * 512;
    const int bk = (fetch_k / kFBK) * L.b_step;
#pragma unroll
    for (int i = 0; i < 2; ++i) fast_buffer_to_lds(L.b_rsrc, sb + i * 1024, L.b_src[i], bk);
}

template <int kRows>
__device__ __forceinline__ void fast_fetch(MC_LDS unsigned char* wr, const FastLane<kRows>& L, int fetch_k) {
    fast_fetch_a<kRows>(wr, L, fetch_k);
    fast_fetch_b<kRows>(wr, L, fetch_k);
}

template <int kRows>
__device__ __forceinline__ mc_u16x8_t fast_read_a(const MC_LDS unsigned char* rd, const FastLane<kRows>& L, int f) {
    return *reinterpret_cast<const MC_LDS mc_u16x8_t*>(rd + L.a_off[f]);
}

template <int kRows>
__device__ __forceinline__ mc_u16x8_t fast_read_b(const MC_LDS unsigned char* rd, const FastLane<kRows>& L, int f) {
    MC_LDS unsigned char* p = const_cast<MC_LDS unsigned char*>(rd);
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(reinterpret_cast<MC_LDS s16x4*>(p + L.b_off[0][f]));
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(reinterpret_cast<MC_LDS s16x4*>(p + L.b_off[1][f]));
    return __builtin_bit_cast(mc_u16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

// Memory phase: fetch A of step `fetch_k` into `wr` and read the operands of
// the step held in `rd` into (av, bv); B of step `fetch_k` is fetched in the
// middle of the compute phase. `rd` and `wr` are distinct stages;
// declaring them __restrict__ gives the LDS reads alias scopes that keep the
// compiler from making them wait for the fetch.
template <int kRows>
__device__ __forceinline__ void fast_memory_phase(const MC_LDS unsigned char* __restrict__ rd,
                                                  MC_LDS unsigned char* __restrict__ wr, const FastLane<kRows>& L,
                                                  int fetch_k, mc_u16x8_t (&av)[FastShape<kRows>::kRowFrags],
                                                  mc_u16x8_t (&bv)[kFColFrags]) {
    fast_fetch_a<kRows>(wr, L, fetch_k);
#pragma unroll
    for (int f = 0; f < FastShape<kRows>::kRowFrags; ++f) av[f] = fast_read_a<kRows>(rd, L, f);
#pragma unroll
    for (int f = 0; f < kFColFrags; ++f) bv[f] = fast_read_b<kRows>(rd, L, f);
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

// Lane l takes the value of lane (l & ~15) | ((l + 8) & 15): a rotation by
// 8 within each row of 16 lanes (DPP row_ror:8).
__device__ __forceinline__ float mc_row_ror8(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), 0x128, 0xf, 0xf, false));
}

// The store of a wave's accumulators, whose first row and column are (row,
// col): lane l = 16 g + i of acc[fi][fj] holds
// C[row + 16 fi + i][col + 16 fj + 4 g + v], v = 0..3, so a store straight
// from one fragment writes 64 bytes in each of 16 rows, half of every
// 128-byte line. Two neighbouring fragments (16 fj = 32 p and 32 p + 16)
// cover 32 columns, whole lines: lanes with i >= 8 of the first swap with
// lanes with i < 8 of the second (a rotation by 8 within each 16-lane row and
// a select), after which one register holds rows 0-7 and the other rows
// 8-15 of the pair, lane l at row 8 h + l % 8 and 16-byte chunk
// l / 16 + 4 ((l / 8) % 2). Each store instruction then writes 8 whole lines.
// kCheck: some rows or columns may be past the matrix edge.
// Non-temporal: every CU stores its tile at the same moment, with its matrix
// units idle until the next tile starts. On one MI355X in one process, at
// 8192^3 with A packed: 782 us with half-line stores, 766 us with whole
// lines; on 4096x14336x4096 393 and 374 us; 708 us at 8192^3 with no store at
// all (a timing-only variant). Plain stores instead of non-temporal ones
// were slower (811 against 777 us with half lines).
template <int kRowFrags, bool kCheck, typename Epilogue>
__device__ __forceinline__ void fast_store(const mc_f32x4_t (&acc)[kRowFrags][kFColFrags], float* __restrict__ c,
                                           int row, int col, int m, int n, int lane, const Epilogue& epilogue) {
    const bool hi = (lane & 8) != 0;
    const int lr = lane & 7;
    const int chunk = (lane >> 4) + (hi ? 4 : 0);
#pragma unroll
    for (int fi = 0; fi < kRowFrags; ++fi) {
#pragma unroll
        for (int p = 0; p < kFColFrags / 2; ++p) {
            const mc_f32x4_t fa = acc[fi][2 * p], fb = acc[fi][2 * p + 1];
            mc_f32x4_t t[2];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float ra = mc_row_ror8(fa[e]), rb = mc_row_ror8(fb[e]);
                t[0][e] = hi ? rb : fa[e];
                t[1][e] = hi ? fb[e] : ra;
            }
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int r = row + fi * 16 + 8 * h + lr;
                const int cc = col + 32 * p + 4 * chunk;
                if (kCheck && (r >= m || cc >= n)) continue;
                const unsigned at = static_cast<unsigned>(static_cast<long long>(r) * n + cc);
                mc_f32x4_t v = t[h];
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = epilogue(v[e], at + e);
                __builtin_nontemporal_store(v, reinterpret_cast<mc_f32x4_t*>(c + static_cast<long long>(r) * n + cc));
            }
        }
    }
}

// One kRows x 256 tile of C at (row0, col0), all of K.
template <bool kBf16, int kRows, bool kPackedA, typename Epilogue>
__device__ __forceinline__ void fast_tile(MC_LDS unsigned char* lds, const unsigned short* __restrict__ a,
                                          const unsigned short* __restrict__ b, float* __restrict__ c, int m, int n,
                                          int k, int row0, int col0, const Epilogue& epilogue) {
    typedef FastShape<kRows> Sh;
    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;

    FastLane<kRows> L;
    L.wave = wave;
    // Row-major A: based at row row0. Packed A: at the row's 256-row band,
    // plus 8 KiB for the second half of a band, the step blocks 16 KiB apart.
    const long long a_base = kPackedA ? static_cast<long long>(row0 / kFBM) * k * kFBM + (row0 % kFBM) * 32
                                      : static_cast<long long>(row0) * k;
    L.a_rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned short*>(a) + a_base, 0, 0x7fffffff, 0x00020000);
    L.a_step = kPackedA ? kFBM * kFBK * 2 : kFBK * 2;
    L.b_rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned short*>(b) + col0, 0, 0x7fffffff, 0x00020000);
    // A: wave w fills the 16-row blocks kFetchA w + i, one per instruction;
    // lane -> (row 16 (kFetchA w + i) + l % 16, chunk l / 16). Rows past the
    // edge are clamped, so every offset is at or past the origin.
#pragma unroll
    for (int i = 0; i < Sh::kFetchA; ++i) {
        if constexpr (kPackedA) {
            // The stage's A bytes as they lie in a step block: 1 KiB per
            // instruction, read linearly.
            L.a_src[i] = (wave * Sh::kFetchA + i) * 1024 + lane * 16;
        } else {
            const int r = (wave * Sh::kFetchA + i) * 16 + (lane & 15);
            const int gr = mc_min16(row0 + r, m - 1);
            L.a_src[i] = 2 * ((gr - row0) * k + (lane >> 4) * 8);
        }
    }
    // B: wave w fills k rows 4 w .. 4 w + 3, two per instruction; lane ->
    // (k row 4 w + 2 i + l / 32, physical chunk l % 32).
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int kr = wave * 4 + i * 2 + (lane >> 5);
        const int lc = (lane & 31) ^ (2 * swz_b(kr));
        const int gc = mc_min16(col0 + lc * 8, n - 8);
        L.b_src[i] = 2 * (kr * n + gc - col0);
    }
    L.b_step = 2 * kFBK * n;
    // Wave (wm, wn) of the 2x4 grid owns rows kRows / 2 wm .., columns 64 wn ...
    const int wr = (wave >> 2) * (kRows / 2), wc = (wave & 3) * 64;
    const int g = lane >> 4;
#pragma unroll
    for (int f = 0; f < Sh::kRowFrags; ++f) L.a_off[f] = (wr + f * 16) * 64 + lane * 16;
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

    mc_f32x4_t acc[Sh::kRowFrags][kFColFrags];
#pragma unroll
    for (int i = 0; i < Sh::kRowFrags; ++i)
#pragma unroll
        for (int j = 0; j < kFColFrags; ++j) acc[i][j] = mc_f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

    const int steps = k / kFBK;
    auto stage = [&](int t) { return lds + (t & (kFStages - 1)) * kFStage; };
    mc_u16x8_t av[Sh::kRowFrags], bv[kFColFrags];
    // Prologue: steps 0..2 landed.
    const int pre = mc_min16(steps, kFStages - 1);
    for (int t = 0; t < pre; ++t) fast_fetch<kRows>(stage(t), L, t * kFBK);
    __builtin_amdgcn_s_waitcnt(0);
    step_barrier();
    // Waves 4-7 start one phase late.
    const bool late = wave >= kFWaves / 2;
    if (late) step_barrier();

    // Every iteration fetches step t+3 into the stage of step t-1, which no
    // wave reads any more (past the last step it fetches the last step again):
    // A in the memory phase, B between the two halves of the MFMAs, which
    // keeps the memory phase shorter than the other group's compute phase
    // (fetching both in the memory phase ran 3% slower at 8192^3). After A of
    // step t+3 this wave has B of t+2, A of t+2 and A of t+3 in flight behind
    // the fetch of t+1 and waits for t+1, which the other group reads two
    // phases later; loads into LDS complete in issue order.
    const int last = (steps - 1) * kFBK;
    for (int t = 0; t < steps; ++t) {
        const int fetch_k = mc_min16((t + 3) * kFBK, last);
        fast_memory_phase<kRows>(stage(t), stage(t + 3), L, fetch_k, av, bv);
        __builtin_amdgcn_s_waitcnt(0x0070 | (2 * Sh::kFetch - 2));  // vmcnt(2 kFetch - 2), lgkmcnt(0)
        step_barrier();
#pragma unroll
        for (int fi = 0; fi < Sh::kRowFrags / 2; ++fi)
#pragma unroll
            for (int fj = 0; fj < kFColFrags; ++fj) acc[fi][fj] = mc_mfma16<kBf16>(bv[fj], av[fi], acc[fi][fj]);
        __builtin_amdgcn_sched_barrier(0);
        fast_fetch_b<kRows>(stage(t + 3), L, fetch_k);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int fi = Sh::kRowFrags / 2; fi < Sh::kRowFrags; ++fi)
#pragma unroll
            for (int fj = 0; fj < kFColFrags; ++fj) acc[fi][fj] = mc_mfma16<kBf16>(bv[fj], av[fi], acc[fi][fj]);
        step_barrier();
    }
    if (!late) step_barrier();
    __builtin_amdgcn_s_waitcnt(0);

    if (row0 + kRows <= m && col0 + kFBN <= n)
        fast_store<Sh::kRowFrags, false>(acc, c, row0 + wr, col0 + wc, m, n, lane, epilogue);
    else
        fast_store<Sh::kRowFrags, true>(acc, c, row0 + wr, col0 + wc, m, n, lane, epilogue);
}

// C = A B with the epilogue mapping each accumulated value v of element
// i = row n + col to what is stored. The tiles are 256x256 in row-major
// order; the grid has one block per tile plus `halves` = gridDim.x - tiles
// more: the last `halves` tiles each run as two blocks of 128 x 256 (rows
// 0-127 and 128-255), so a last round that would fill at most half of the
// CUs (896 tiles on 256 CUs: 3 rounds and 128 tiles) runs at half the work
// per block on all of them (mchip_mfma16_fast_grid picks the count). Every C
// element gets the same MFMA sequence either way, so the results are the
// same bits.
template <bool kBf16, bool kPackedA, typename Epilogue>
__device__ __forceinline__ void mc_gemm16_fast(const unsigned short* __restrict__ a, const unsigned short* __restrict__ b,
                                               float* __restrict__ c, int m, int n, int k, const Epilogue& epilogue) {
    __shared__ __attribute__((aligned(1024))) unsigned char smem[kFStages * kFStage];
    MC_LDS unsigned char* lds = (MC_LDS unsigned char*)(smem);  // generic -> LDS address space

    const int tiles_n = (n + kFBN - 1) / kFBN;
    const int tiles = ((m + kFBM - 1) / kFBM) * tiles_n;
    const int halves = static_cast<int>(gridDim.x) - tiles;
    const int full = tiles - halves;
    const int bid = static_cast<int>(blockIdx.x);
    if (bid < full) {
        const int tm = bid / tiles_n, tn = bid % tiles_n;
        fast_tile<kBf16, kFBM, kPackedA>(lds, a, b, c, m, n, k, tm * kFBM, tn * kFBN, epilogue);
    } else {
        const int t = full + (bid - full) / 2, half = (bid - full) % 2;
        const int tm = t / tiles_n, tn = t % tiles_n;
        const int row0 = tm * kFBM + half * (kFBM / 2);
        // In a last tile row of at most 128 rows the second half has no row
        // of C: it has nothing to store, and its clamped rows would sit
        // before its origin (fetch offsets below zero).
        if (row0 >= m) return;
        fast_tile<kBf16, kFBM / 2, kPackedA>(lds, a, b, c, m, n, k, row0, tn * kFBN, epilogue);
    }
}
