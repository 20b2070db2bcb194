// FP32 GEMM body for narrow tiles: C tiles of 16 kRG rows x 16 kVec columns
// (32x64, 16x64 or 16x32) on v_mfma_f32_16x16x4f32, for products too small
// or too thin to fill the chip
// with the ring body's 128x128 and 256x256 tiles (M <= 16, where B is read
// once and HBM is the bound; and products of a few million outputs or
// fewer, where small tiles give every CU a share without deep K splits).
// Shared by the ahead-of-time kernels (identity epilogue) and the GEMMs
// compiled at run time with a fused elementwise epilogue. No headers, so
// hipRTC compiles it as is; it uses the split-K helpers
// of gemm_split_arrival.h, which the includer puts before it.
//
// No LDS staging of operands: each wave loads its A and B fragments straight
// from global memory (L2 for data other waves share) into registers, all the
// loads of a batch of K before the batch's MFMAs, so a wave keeps many loads
// in flight and each group's MFMAs start as soon as that group has landed.
//
// Decomposition: logical block (x, y, z) owns columns 16 V x .. 16 V x +
// 16 V - 1, rows 16 kRG z .., and the y-th of `depth` ranges of K (k_split
// each); the grid is one-dimensional, ceil(n / 16 V) ceil(m / 16 kRG) depth
// blocks (mapped to logical blocks XCD by XCD, below); its kW
// waves cut that range into consecutive pieces, one accumulator set each.
// Lane l of a wave has k slot s = l / 16 and index c = l % 16. For each group
// of 16 k from kg the lane loads (V = kVec, 4 or 2 columns per lane)
//   A[16 r + c][kg + 4s .. kg + 4s + 3]              for row group r < kRG
//   B[kg + 4s + e][col0 + V c .. col0 + V c + V - 1] for e = 0..3
// and MFMA (r, e, j) takes A load r's element e and B load e's element j:
// its k slot s is k = kg + 4s + e and its column slot c is column
// col0 + V c + j, so accumulator (r, j) holds, in lane l, C[16 r + 4s + v]
// [col0 + V c + j] for v = 0..3. The waves' tiles are then added in wave
// order through LDS (a fixed order), and the block stores its tile to C
// through the epilogue, or, with several K ranges, to its range's partial:
// with `counters`, the last of the tile's blocks to finish then adds the
// ranges' partials in range order and stores C through the epilogue
// (mc_split_last_arrival); without, a separate launch adds them.
//
// Requirements (checked by the host): k and k_split multiples of 16, n a
// multiple of kVec (the host asks for 4), A and B 16-byte aligned (C and
// the partials may be at any float address; counters: one zeroed unsigned
// per tile, in tile order). Rows past m read row m - 1 and
// columns past n the last column chunk (every load in bounds); what they
// produce is not stored.
#pragma once

typedef float mc_nw_f32x4 __attribute__((ext_vector_type(4)));
typedef float mc_nw_f32x2 __attribute__((ext_vector_type(2)));

template <int N>
struct McNarrowUnits {
    static constexpr int value = N;
};

// B loads of kVec floats per lane (a 16-lane row segment of 16 kVec floats).
template <int kVec>
struct McNarrowVec;
template <>
struct McNarrowVec<4> {
    typedef mc_nw_f32x4 type;
};
template <>
struct McNarrowVec<2> {
    typedef mc_nw_f32x2 type;
};

// A configuration: kRG row groups of 16, kVec columns per lane and load
// (tiles of 16 kVec columns), kW waves, up to kU groups of 16 k per batch of
// loads; kStreamB: B is read by one tile row only (M <= 16), so its loads
// are non-temporal (a read-only stream reached 7.1 TB/s with them against
// 6.3 TB/s without on an MI355X). kRedRows: rows of the LDS array the waves
// add their tiles through (at least kRows); more than kRows only to keep a
// second block off the CU (LDS is 160 KiB per CU).
template <int kRG_, int kVec_, int kW_, int kU_, bool kStreamB_, int kRedRows_ = 16 * kRG_>
struct McNarrowCfg {
    static constexpr int kRG = kRG_, kVec = kVec_, kW = kW_, kU = kU_;
    static constexpr bool kStreamB = kStreamB_;
    static constexpr int kRows = 16 * kRG, kCols = 16 * kVec, kThreads = 64 * kW;
    static constexpr int kRedRows = kRedRows_;
    static_assert(kRedRows >= kRows, "the reduction holds a whole tile");
};

// The configurations the library runs, 4 waves each, batches of up to 2
// groups: 16x64 tiles for M <= 16 (B streamed), 32x64 tiles, and for
// short-K products that these would leave with half the CUs idle, 16x64 and
// 16x32 tiles. At one K range every configuration adds the same products in
// the same order (per element: the 4 waves' pieces of K in wave order, each
// a chain of 16x16x4 MFMAs), so they give the same bits.
using McNarrow16 = McNarrowCfg<1, 4, 4, 2, true>;
using McNarrow32 = McNarrowCfg<2, 4, 4, 2, false>;
using McNarrow16x64 = McNarrowCfg<1, 4, 4, 2, false>;
using McNarrow16x32 = McNarrowCfg<1, 2, 4, 2, false>;
// 64x64 tiles: each operand byte a wave loads feeds 64 MFMAs per 16 k
// where 32x64 tiles feed 32 per 6 loads (1024^3 as 256 unsplit tiles). One
// block per CU: its 96 KiB reduction array leaves no room for a second.
// With 512 tiles (two per CU, 1024x2048x512) two co-resident blocks took
// 31-36 us against 22.5 us for one block per CU in two rounds.
using McNarrow64 = McNarrowCfg<4, 4, 4, 2, false, 96>;

// A 16- or 8-byte buffer load at (voffset + soffset) from the resource's
// base; kStream: non-temporal (the slc bit: a read-only stream reached 7.1
// TB/s with non-temporal loads against 6.3 TB/s without on an MI355X).
template <typename T, bool kStream>
__device__ __forceinline__ T mc_narrow_load(__amdgpu_buffer_rsrc_t rsrc, int voffset, int soffset) {
    constexpr int kAux = kStream ? 2 : 0;
    if constexpr (sizeof(T) == 16)
        return __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b128(rsrc, voffset, soffset, kAux));
    else
        return __builtin_bit_cast(T, __builtin_amdgcn_raw_buffer_load_b64(rsrc, voffset, soffset, kAux));
}

// One batch of a wave's operands: kU groups of 16 k.
template <class Cfg>
struct McNarrowRegs {
    typedef typename McNarrowVec<Cfg::kVec>::type BV;
    mc_nw_f32x4 a[Cfg::kU][Cfg::kRG];
    BV b[Cfg::kU][4];
};

// The tile of C at (row0, col0) and its K range [kb, ke), accumulated by
// this block; the epilogue maps each value v of flat element i to what is
// stored (out = C), or the raw sums go to `out` (a partial), added in the
// launch when `counters` is given (not null).
template <class Cfg, typename Epilogue>
__device__ __forceinline__ void mc_gemm_f32_narrow(const float* __restrict__ a, const float* __restrict__ b,
                                                   float* __restrict__ c, int m, int n, int k, int k_split,
                                                   int depth, float* __restrict__ partial, unsigned* __restrict__ counters,
                                                   const Epilogue& epilogue) {
    constexpr int kRG = Cfg::kRG, kW = Cfg::kW, kVec = Cfg::kVec, kU = Cfg::kU;
    typedef typename McNarrowVec<kVec>::type BV;
    __shared__ BV red[kW][Cfg::kRedRows][16];  // [wave][row][column chunk]
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
    const int s = lane >> 4, cl = lane & 15;
    // The grid is one-dimensional: block L runs on XCD L % 8 (the hardware
    // hands consecutive workgroups to the 8 XCDs in turn). With the count a
    // multiple of 8, XCD x takes the x-th contiguous eighth of the blocks in
    // (column tile, row tile, K range) order, so the blocks sharing an L2
    // share K ranges of A and B (one range per XCD when there are 8).
    const int tiles_n = (n + Cfg::kCols - 1) / Cfg::kCols;
    const int tiles_m = (m + Cfg::kRows - 1) / Cfg::kRows;
    const int total = static_cast<int>(gridDim.x);
    const int L = static_cast<int>(blockIdx.x);
    const int q = total % 8 == 0 ? (L % 8) * (total / 8) + L / 8 : L;
    const int bx = q % tiles_n, bz = (q / tiles_n) % tiles_m, by = q / (tiles_n * tiles_m);
    const int col0 = bx * Cfg::kCols;
    const int row0 = bz * Cfg::kRows;
    const int colc = col0 + kVec * cl < n ? col0 + kVec * cl : n - kVec;

    // This wave's K range: the block's range cut into kW pieces of whole
    // 16-k groups (the last pieces may be empty).
    const int kb = by * k_split;
    const int ke = kb + k_split < k ? kb + k_split : k;
    const int groups = (ke - kb) / 16;
    const int per = (groups + kW - 1) / kW;
    const int g0 = wave * per < groups ? wave * per : groups;
    const int g1 = g0 + per < groups ? g0 + per : groups;

    // Operands through buffer loads: bases at the block's origin in A (row
    // row0, column kb) and B (row kb, column col0) in scalar registers, the
    // lane's byte offset from them in a vector register, the group's offset
    // (64 g bytes in A, 64 g n in B) in a scalar one, so no vector
    // instruction computes a load address (the host keeps every offset below
    // 2^31: mchip_f32_narrow_plan).
    const __amdgpu_buffer_rsrc_t a_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(a) + static_cast<long long>(row0) * k + kb, 0, 0x7fffffff, 0x00020000);
    const __amdgpu_buffer_rsrc_t b_rsrc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(b) + static_cast<long long>(kb) * n + col0, 0, 0x7fffffff, 0x00020000);
    int a_off[kRG];
#pragma unroll
    for (int r = 0; r < kRG; ++r) {
        const int row = row0 + 16 * r + cl < m ? row0 + 16 * r + cl : m - 1;
        a_off[r] = 4 * ((row - row0) * k + 4 * s);
    }
    const int b_off = 4 * (4 * s * n + colc - col0);
    const int b_row = 4 * n;  // bytes per row of B

    mc_nw_f32x4 acc[kRG][kVec] = {};
    // Loads of `units` groups from group g into x, then (after a scheduling
    // barrier: left to itself the scheduler interleaves each load with the
    // MFMAs that use it and waits for it there) nothing else.
    auto load = [&](McNarrowRegs<Cfg>& x, int g, auto units) {
        constexpr int kN = decltype(units)::value;
#pragma unroll
        for (int u = 0; u < kN; ++u) {
#pragma unroll
            for (int r = 0; r < kRG; ++r) x.a[u][r] = mc_narrow_load<mc_nw_f32x4, false>(a_rsrc, a_off[r], 64 * (g + u));
#pragma unroll
            for (int e = 0; e < 4; ++e)
                x.b[u][e] = mc_narrow_load<BV, Cfg::kStreamB>(b_rsrc, b_off, (16 * (g + u) + e) * b_row);
        }
        __builtin_amdgcn_sched_barrier(0);
    };
    // The MFMAs of `units` groups held in x: MFMA (u, e, r, j) multiplies A
    // load (u, r)'s element e by B load (u, e)'s element j.
    auto compute = [&](const McNarrowRegs<Cfg>& x, auto units) {
        constexpr int kN = decltype(units)::value;
#pragma unroll
        for (int u = 0; u < kN; ++u)
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int r = 0; r < kRG; ++r)
#pragma unroll
                    for (int j = 0; j < kVec; ++j)
                        acc[r][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(x.a[u][r][e], x.b[u][e][j], acc[r][j], 0, 0, 0);
        __builtin_amdgcn_sched_barrier(0);
    };
    // Whole batches, software-pipelined over two register sets: the loads of
    // batch i + 1 are issued before the MFMAs of batch i, so the wave keeps
    // loads in flight while its matrix core works. Every load is issued
    // unconditionally where it is issued (the last batch is peeled off): a
    // load under a condition would make the compiler wait for all loads
    // before the next MFMA. A batch is kU groups when each wave has 32 groups
    // or more and the block has one of several K ranges or 16-row tiles,
    // else one group: a short piece gains more from MFMAs that start after
    // one group's loads than from more loads in flight. Measured on an MI355X
    // (batches of 1 / 2 / 4 groups): 256x2048x512 on 32x64 tiles 7.8 / 9.0 /
    // 10.5 us, 512^3 on 16x64 tiles 5.0 / 5.2 / 6.1 us, 16x4096x4096 streamed
    // in 4 K ranges 13.4 / 13.9 / 14.4 us; with 32 groups per wave:
    // 256x256x16384 on 32x64 tiles in 8 ranges 21.7 / 21.0 / 24.9 us,
    // 256x512x2048 on 16x32 tiles 10.2 / 9.8 / 10.1 us, but 1024x512x2048 on
    // 32x64 tiles unsplit 18.5 / 20.2 us. The batching does not change the
    // order of the adds.
    McNarrowRegs<Cfg> x0, x1;
    auto pipeline = [&](auto units) {
        constexpr int kN = decltype(units)::value;
        const int batches = (g1 - g0) / kN;
        if (batches > 0) {
            int i = 0;
            load(x0, g0, units);
            for (; i + 2 < batches; i += 2) {
                load(x1, g0 + (i + 1) * kN, units);
                compute(x0, units);
                load(x0, g0 + (i + 2) * kN, units);
                compute(x1, units);
            }
            if (batches - i == 2) {
                load(x1, g0 + (i + 1) * kN, units);
                compute(x0, units);
                compute(x1, units);
            } else {
                compute(x0, units);
            }
        }
        for (int g = g0 + batches * kN; g < g1; ++g) {
            load(x0, g, McNarrowUnits<1>{});
            compute(x0, McNarrowUnits<1>{});
        }
    };
    if (kU > 1 && per >= 32 && (depth > 1 || kRG == 1)) {
        pipeline(McNarrowUnits<kU>{});
    } else {
        pipeline(McNarrowUnits<1>{});
    }

    // Lane l holds rows 16 r + 4s + v of column chunk cl.
#pragma unroll
    for (int r = 0; r < kRG; ++r)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            BV o;
#pragma unroll
            for (int j = 0; j < kVec; ++j) o[j] = acc[r][j][v];
            red[wave][16 * r + 4 * s + v][cl] = o;
        }
    __syncthreads();
    // The tile's chunks, summed over the waves in wave order.
    const bool raw = depth > 1;
    float* __restrict__ out = raw ? partial + static_cast<long long>(by) * m * n : c;
    // C or a partial may sit at any 4-byte address (a caller's workspace):
    // then a chunk is stored float by float, the same values. Partials that
    // this launch adds go out as device-scope stores (mc_split_store).
    const bool fold = raw && counters != nullptr;
    const bool vec_out = (reinterpret_cast<unsigned long long>(out) & (sizeof(BV) - 1)) == 0;
    // A lane's chunks (kRows 16 / kThreads of them, 1 to 4): all summed and
    // through the epilogue before the first store, so the epilogue's operand
    // loads of every chunk are in flight together, and a per-column operand
    // (a bias: every chunk of a lane is in the same columns) is loaded once;
    // chunk by chunk, the compiler loaded it again and waited for it in each
    // chunk, after the previous chunk's store.
    constexpr int kChunks = Cfg::kRows * 16 / Cfg::kThreads;
    static_assert(kChunks * Cfg::kThreads == Cfg::kRows * 16, "a whole number of chunks per lane");
    BV sums[kChunks];
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
        const int t = static_cast<int>(threadIdx.x) + i * Cfg::kThreads;
        const int r = t >> 4, ch = t & 15;
        BV sum = red[0][r][ch];
#pragma unroll
        for (int w = 1; w < kW; ++w) sum += red[w][r][ch];
        const int row = row0 + r, col = col0 + kVec * ch;
        if (!raw && row < m && col < n) {
            const long long at = static_cast<long long>(row) * n + col;
#pragma unroll
            for (int j = 0; j < kVec; ++j) sum[j] = epilogue(sum[j], static_cast<unsigned>(at + j));
        }
        sums[i] = sum;
    }
#pragma unroll
    for (int i = 0; i < kChunks; ++i) {
        const int t = static_cast<int>(threadIdx.x) + i * Cfg::kThreads;
        const int r = t >> 4, ch = t & 15;
        const int row = row0 + r, col = col0 + kVec * ch;
        if (row >= m || col >= n) continue;
        const long long at = static_cast<long long>(row) * n + col;
        if (fold) {
#pragma unroll
            for (int j = 0; j < kVec; ++j) mc_split_store(out + at + j, sums[i][j]);
        } else if (vec_out) {
            *reinterpret_cast<BV*>(out + at) = sums[i];
        } else {
#pragma unroll
            for (int j = 0; j < kVec; ++j) out[at + j] = sums[i][j];
        }
    }
    if (!fold) return;

    // The last block of the tile adds the ranges' partials, range 0 first (a
    // lane issues its loads of 8 ranges before it adds them), and stores C.
    __shared__ int last_flag;
    if (!mc_split_last_arrival(counters + bz * tiles_n + bx, depth, &last_flag)) return;
    const long long plane = static_cast<long long>(m) * n;
    const bool vec_c = (reinterpret_cast<unsigned long long>(c) & (sizeof(BV) - 1)) == 0;
    constexpr int kChunk = 8;
    for (int t = threadIdx.x; t < Cfg::kRows * 16; t += Cfg::kThreads) {
        const int r = t >> 4, ch = t & 15;
        const int row = row0 + r, col = col0 + kVec * ch;
        if (row >= m || col >= n) continue;
        const long long at = static_cast<long long>(row) * n + col;
        auto load = [&](int z) {
            const float* p = partial + z * plane + at;
            BV x;
#pragma unroll
            for (int j = 0; j < kVec; ++j) x[j] = mc_split_load(p + j);
            return x;
        };
        BV sum = load(0);
        for (int z0 = 1; z0 < depth; z0 += kChunk) {
            BV x[kChunk];
#pragma unroll
            for (int i = 0; i < kChunk; ++i) x[i] = load(z0 + i < depth ? z0 + i : depth - 1);
#pragma unroll
            for (int i = 0; i < kChunk; ++i)
                if (z0 + i < depth) sum += x[i];
        }
#pragma unroll
        for (int j = 0; j < kVec; ++j) sum[j] = epilogue(sum[j], static_cast<unsigned>(at + j));
        if (vec_c) {
            *reinterpret_cast<BV*>(c + at) = sum;
        } else {
#pragma unroll
            for (int j = 0; j < kVec; ++j) c[at + j] = sum[j];
        }
    }
}
