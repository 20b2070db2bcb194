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

#include <atomic>

#include "gemm_mfma16_fast.h"

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
// The body lives in gemm_mfma16_fast.h (also compiled at run time with fused
// epilogues); here it is instantiated with the identity epilogue.

template <bool kBf16, bool kPackedA>
__global__ void __launch_bounds__(kFThreads, 1) matmul_mfma16_fast(const unsigned short* __restrict__ a,
                                                                   const unsigned short* __restrict__ b,
                                                                   float* __restrict__ c, int m, int n, int k) {
    mc_gemm16_fast<kBf16, kPackedA>(a, b, c, m, n, k, McGemm16Store{});
}

// The fast path takes 16-bit A and B with K a multiple of 64, N a multiple
// of 8 (every 16-byte B chunk wholly inside or outside a row), A, B and C
// 16-byte aligned, and no split.
bool fast_eligible(const void* a, const void* b, const float* c, int m, int n, int k, int splits) {
    const auto al = [](const void* p) { return reinterpret_cast<std::uintptr_t>(p) % 16 == 0; };
    return splits <= 1 && mchip_mfma16_fast_fits(m, n, k) && al(a) && al(b) && al(c);
}

// CUs of the current device, asked once per device.
int device_cus() {
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

template <bool kBf16, bool kPackedA = false>
int launch_fast(const void* a, const void* b, float* c, int m, int n, int k, hipStream_t stream) {
    const long long tiles = static_cast<long long>((m + kFBM - 1) / kFBM) * ((n + kFBN - 1) / kFBN);
    if (tiles > 0x3fffffffLL) return hipErrorInvalidValue;
    const unsigned grid = mchip_mfma16_fast_grid(m, n, device_cus());
    hipLaunchKernelGGL((matmul_mfma16_fast<kBf16, kPackedA>), dim3(grid), dim3(kFThreads), 0, stream,
                       static_cast<const unsigned short*>(a), static_cast<const unsigned short*>(b), c, m, n, k);
    return hipGetLastError();
}

// ------------------------------------------------------------ packed A
//
// One lane per 16-byte chunk of the packed layout (gemm_mfma16_fast.h): 8
// consecutive k of one row. Consecutive lanes take consecutive chunks, so a
// wave writes 1 KiB of consecutive memory and reads 16 rows x 4 chunks
// (64 bytes of 16-bit A, 128 of fp32 A, per row). Rows past M are zeros.
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

struct PackedChunk {
    int row, kk;
};

__device__ __forceinline__ PackedChunk packed_chunk(long long q, int steps) {
    const long long blk = q >> 10;
    const int w = static_cast<int>(q & 1023);
    const int band = static_cast<int>(blk / steps), step = static_cast<int>(blk % steps);
    return {band * kFBM + (w >> 6) * 16 + (w & 15), step * kFBK + ((w >> 4) & 3) * 8};
}

// kVec: `in` 16-byte aligned (one 16-byte load per chunk), else 8 loads of
// 2 bytes.
template <bool kVec>
__global__ void __launch_bounds__(256) pack_a16_kernel(const unsigned short* __restrict__ in, u32x4* __restrict__ out,
                                                       int m, int k, long long chunks) {
    const int steps = k / kFBK;
    const long long stride = static_cast<long long>(gridDim.x) * 256;
    for (long long q = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x; q < chunks; q += stride) {
        const PackedChunk p = packed_chunk(q, steps);
        u32x4 v = {0u, 0u, 0u, 0u};
        if (p.row < m) {
            const unsigned short* src = in + static_cast<long long>(p.row) * k + p.kk;
            if constexpr (kVec) {
                v = *reinterpret_cast<const u32x4*>(src);
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j) v[j] = src[2 * j] | (static_cast<unsigned>(src[2 * j + 1]) << 16);
            }
        }
        out[q] = v;
    }
}

// fp32 A at any 4-byte address rounded and packed, 8 loads of 4 bytes per
// chunk. The rounding is mchip_convert_f32's.
template <bool kBf16>
__global__ void __launch_bounds__(256) convert_pack_a_kernel(const float* __restrict__ in, u32x4* __restrict__ out,
                                                             int m, int k, long long chunks) {
    const int steps = k / kFBK;
    const long long stride = static_cast<long long>(gridDim.x) * 256;
    for (long long q = static_cast<long long>(blockIdx.x) * 256 + threadIdx.x; q < chunks; q += stride) {
        const PackedChunk p = packed_chunk(q, steps);
        u32x4 v = {0u, 0u, 0u, 0u};
        if (p.row < m) {
            const float* src = in + static_cast<long long>(p.row) * k + p.kk;
#pragma unroll
            for (int j = 0; j < 4; ++j)
                v[j] = to_bits<kBf16>(src[2 * j]) | (static_cast<unsigned>(to_bits<kBf16>(src[2 * j + 1])) << 16);
        }
        out[q] = v;
    }
}

// fp32 A rounded and packed through LDS, for 16-byte aligned A: a block
// takes kSteps K steps of one 256-row band. It reads them as rows of
// kSteps x 128 contiguous bytes (a wave reads 1 KiB: 2 or 4 rows), writes the
// rounded values into the band's packed blocks in LDS, then writes those out
// as 1 KiB per wave instruction. (Reading straight into packed order, a wave
// read 64 bytes from each of 16 rows: 4.4 TB/s on an MI355X against 6.0 for
// the plain rounding.) In LDS each 16-byte chunk's row slot is XORed with
// (step, chunk) % 16, which spreads a wave's 8-byte writes over the banks
// (unswizzled, all of a row's 32 writes fall in 2 of the 64 banks); the
// read-out undoes it, 16 lanes reading 256 contiguous bytes.
template <bool kBf16, int kSteps>
__global__ void __launch_bounds__(256) convert_pack_a_lds(const f32x4* __restrict__ in, u32x4* __restrict__ out, int m,
                                                          int k, long long regions) {
    __shared__ u32x4 tile[kSteps * 1024];
    unsigned char* lds = reinterpret_cast<unsigned char*>(tile);
    constexpr int kF4PerRow = kSteps * 8;
    const int steps = k / kFBK;
    const int per_band = steps / kSteps;
    const int tid = static_cast<int>(threadIdx.x);
    for (long long reg = blockIdx.x; reg < regions; reg += gridDim.x) {
        const int band = static_cast<int>(reg / per_band), s0 = static_cast<int>(reg % per_band) * kSteps;
        // Eight 16-byte loads in flight per lane, then their LDS writes.
        for (int i0 = 0; i0 < kF4PerRow; i0 += 8) {
            f32x4 v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int f = (i0 + j) * 256 + tid;
                const int grow = band * kFBM + f / kF4PerRow;
                v[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                if (grow < m) {
                    v[j] = __builtin_nontemporal_load(in + (static_cast<long long>(grow) * k + s0 * kFBK) / 4 +
                                                      f % kF4PerRow);
                }
            }
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int f = (i0 + j) * 256 + tid;
                const int row = f / kF4PerRow, k4 = f % kF4PerRow;
                const int sl = k4 >> 3, c = (k4 >> 1) & 3, eh = k4 & 1;
                const int slot = (row & 15) ^ ((sl * 4 + c) & 15);
                const int at = sl * 16384 + (row >> 4) * 1024 + c * 256 + slot * 16 + eh * 8;
                typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
                const u32x2 w = {to_bits<kBf16>(v[j][0]) | (static_cast<unsigned>(to_bits<kBf16>(v[j][1])) << 16),
                                 to_bits<kBf16>(v[j][2]) | (static_cast<unsigned>(to_bits<kBf16>(v[j][3])) << 16)};
                *reinterpret_cast<u32x2*>(lds + at) = w;
            }
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < kSteps * 4; ++i) {
            const int q = i * 256 + tid;
            const int sl = q >> 10, w = q & 1023, c = (w >> 4) & 3;
            const int slot = (w & 15) ^ ((sl * 4 + c) & 15);
            const u32x4 v = *reinterpret_cast<const u32x4*>(lds + sl * 16384 + (w >> 6) * 1024 + c * 256 + slot * 16);
            out[(static_cast<long long>(band) * steps + s0 + sl) * 1024 + w] = v;
        }
        __syncthreads();
    }
}

unsigned pack_blocks(long long chunks) {
    return static_cast<unsigned>(std::max<long long>(1, std::min<long long>((chunks + 255) / 256, 16384)));
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

// The same rounding on 16-byte-aligned `in` and 8-byte-aligned `out`: a lane
// reads a float4 and writes its four 16-bit values as one 8-byte store, for
// kConvertItems float4s spaced one block apart (each wave instruction reads
// 1 KiB and writes 512 bytes of consecutive memory). Elements past the last
// whole float4 are done one by one by the first block.
constexpr int kConvertItems = 4;

template <bool kBf16>
__global__ void __launch_bounds__(256) convert_vec_kernel(const f32x4* __restrict__ in, u16x4* __restrict__ out,
                                                          std::size_t groups, const float* __restrict__ tail_in,
                                                          unsigned short* __restrict__ tail_out, int tail) {
    const std::size_t span = static_cast<std::size_t>(256) * kConvertItems;
    const std::size_t stride = static_cast<std::size_t>(gridDim.x) * span;
    for (std::size_t base = static_cast<std::size_t>(blockIdx.x) * span + threadIdx.x; base < groups; base += stride) {
        f32x4 v[kConvertItems];
#pragma unroll
        for (int j = 0; j < kConvertItems; ++j) {
            const std::size_t g = base + static_cast<std::size_t>(j) * 256;
            if (g < groups) v[j] = __builtin_nontemporal_load(in + g);
        }
#pragma unroll
        for (int j = 0; j < kConvertItems; ++j) {
            const std::size_t g = base + static_cast<std::size_t>(j) * 256;
            if (g < groups) {
                const u16x4 r = {to_bits<kBf16>(v[j][0]), to_bits<kBf16>(v[j][1]), to_bits<kBf16>(v[j][2]),
                                 to_bits<kBf16>(v[j][3])};
                out[g] = r;
            }
        }
    }
    if (blockIdx.x == 0 && static_cast<int>(threadIdx.x) < tail) {
        tail_out[threadIdx.x] = to_bits<kBf16>(tail_in[threadIdx.x]);
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

extern "C" long long mchip_packed_a16_elements(int m, int k) {
    if (m < 1 || k < 1) return 0;
    return static_cast<long long>((m + kFBM - 1) / kFBM) * kFBM * k;
}

extern "C" int mchip_pack_a16(const void* a, void* packed, int m, int k, void* stream) {
    if (m < 1 || k < 1 || k % (2 * kFBK) != 0 || !aligned(a, 2) || !aligned(packed, 16)) return hipErrorInvalidValue;
    const long long chunks = mchip_packed_a16_elements(m, k) / 8;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const auto* in = static_cast<const unsigned short*>(a);
    if (aligned(a, 16)) {
        hipLaunchKernelGGL(pack_a16_kernel<true>, dim3(pack_blocks(chunks)), dim3(256), 0, s, in,
                           static_cast<u32x4*>(packed), m, k, chunks);
    } else {
        hipLaunchKernelGGL(pack_a16_kernel<false>, dim3(pack_blocks(chunks)), dim3(256), 0, s, in,
                           static_cast<u32x4*>(packed), m, k, chunks);
    }
    return hipGetLastError();
}

extern "C" int mchip_convert_pack_a_f32(int dtype, const float* a, void* packed, int m, int k, void* stream) {
    if (dtype != MCHIP_DTYPE_BF16 && dtype != MCHIP_DTYPE_F16) return hipErrorInvalidValue;
    if (m < 1 || k < 1 || k % (2 * kFBK) != 0 || !aligned(a, 4) || !aligned(packed, 16)) return hipErrorInvalidValue;
    const long long chunks = mchip_packed_a16_elements(m, k) / 8;
    hipStream_t s = static_cast<hipStream_t>(stream);
    auto* out = static_cast<u32x4*>(packed);
    const dim3 grid(pack_blocks(chunks));
    const bool vec = aligned(a, 16);
    if (vec) {
        // Regions of 4 K steps of a band where they tile K, else 2 (K is a
        // multiple of 64); a block per region, up to 8192 blocks that loop.
        const int steps = k / kFBK;
        const bool four = steps % 4 == 0;
        const long long regions = mchip_packed_a16_elements(m, k) / (kFBM * kFBK) / (four ? 4 : 2);
        const dim3 rgrid(static_cast<unsigned>(std::max<long long>(1, std::min<long long>(regions, 8192))));
        const f32x4* in = reinterpret_cast<const f32x4*>(a);
        if (dtype == MCHIP_DTYPE_BF16 && four) {
            hipLaunchKernelGGL((convert_pack_a_lds<true, 4>), rgrid, dim3(256), 0, s, in, out, m, k, regions);
        } else if (dtype == MCHIP_DTYPE_BF16) {
            hipLaunchKernelGGL((convert_pack_a_lds<true, 2>), rgrid, dim3(256), 0, s, in, out, m, k, regions);
        } else if (four) {
            hipLaunchKernelGGL((convert_pack_a_lds<false, 4>), rgrid, dim3(256), 0, s, in, out, m, k, regions);
        } else {
            hipLaunchKernelGGL((convert_pack_a_lds<false, 2>), rgrid, dim3(256), 0, s, in, out, m, k, regions);
        }
    } else if (dtype == MCHIP_DTYPE_BF16) {
        hipLaunchKernelGGL((convert_pack_a_kernel<true>), grid, dim3(256), 0, s, a, out, m, k, chunks);
    } else {
        hipLaunchKernelGGL((convert_pack_a_kernel<false>), grid, dim3(256), 0, s, a, out, m, k, chunks);
    }
    return hipGetLastError();
}

extern "C" int mchip_launch_matmul_lowp_packed(int kernel, int dtype, const void* a_packed, const void* b, float* c,
                                               int m, int n, int k, void* stream) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (m < 1 || n < 1 || k < 1) return hipErrorInvalidValue;
    if (kernel == kTensorCoreTf32) return hipErrorNotSupported;
    if (!fast_eligible(a_packed, b, c, m, n, k, 1)) return hipErrorInvalidValue;
    if (kernel == kTensorCoreBf16 && dtype == MCHIP_DTYPE_BF16) return launch_fast<true, true>(a_packed, b, c, m, n, k, s);
    if (kernel == kTensorCoreF16 && dtype == MCHIP_DTYPE_F16) return launch_fast<false, true>(a_packed, b, c, m, n, k, s);
    return hipErrorInvalidValue;
}

extern "C" int mchip_tensor_core_k_ranges(int k, int splits) {
    if (k < 1) return 0;
    const int k_split = split_len(k, splits, kBK);
    return std::max(1, (k + k_split - 1) / k_split);
}

extern "C" int mchip_mfma16_fast_fits(int m, int n, int k) {
    if (m < 1 || n < 8 || k < 1 || k % (2 * kFBK) != 0 || n % 8 != 0) return 0;
    return 2LL * kFBM * k < (1LL << 31) && 2LL * (static_cast<long long>(k) + kFBK) * n < (1LL << 31);
}

extern "C" unsigned mchip_mfma16_fast_grid(int m, int n, int cu_count) {
    const long long tiles = static_cast<long long>((m + kFBM - 1) / kFBM) * ((n + kFBN - 1) / kFBN);
    const long long rest = cu_count > 0 ? tiles % cu_count : 0;
    const long long halves = rest != 0 && 2 * rest <= cu_count ? rest : 0;
    return static_cast<unsigned>(tiles + halves);
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
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (count == 0) return hipSuccess;
    if (reinterpret_cast<std::uintptr_t>(in) % 16 == 0 && reinterpret_cast<std::uintptr_t>(out) % 8 == 0) {
        const std::size_t groups = count / 4;
        const int tail = static_cast<int>(count % 4);
        const std::size_t per_block = static_cast<std::size_t>(256) * kConvertItems;
        const unsigned blocks =
            static_cast<unsigned>(std::max<std::size_t>(1, std::min<std::size_t>((groups + per_block - 1) / per_block, 8192)));
        const float* tail_in = in + groups * 4;
        unsigned short* tail_out = static_cast<unsigned short*>(out) + groups * 4;
        if (dtype == MCHIP_DTYPE_BF16) {
            hipLaunchKernelGGL(convert_vec_kernel<true>, dim3(blocks), dim3(256), 0, s,
                               reinterpret_cast<const f32x4*>(in), static_cast<u16x4*>(out), groups, tail_in, tail_out,
                               tail);
        } else {
            hipLaunchKernelGGL(convert_vec_kernel<false>, dim3(blocks), dim3(256), 0, s,
                               reinterpret_cast<const f32x4*>(in), static_cast<u16x4*>(out), groups, tail_in, tail_out,
                               tail);
        }
        return hipGetLastError();
    }
    const unsigned blocks = static_cast<unsigned>(std::max<std::size_t>(1, std::min<std::size_t>((count + 255) / 256, 8192)));
    hipLaunchKernelGGL(convert_kernel, dim3(blocks), dim3(256), 0, s, in, static_cast<unsigned short*>(out), count,
                       dtype == MCHIP_DTYPE_BF16 ? 1 : 0);
    return hipGetLastError();
}
