#pragma once

// Generates gfx950 HIP C++ for one elementwise node (a fused program, or a
// single op wrapped as one). Plain C++ with no HIP headers, so it is built
// and tested without a GPU. It takes the place of the reference's
// src/cuda/codegen.hpp:15-40 with the same contract:
//
//   extern "C" __global__ void mc_elementwise(float* out, const float* in0, ..., unsigned n)
//
// where `n` counts 16-byte vectors of 4 floats when the kernel is vectorised
// and single floats otherwise. Shapes are known when the graph is compiled,
// so broadcast index math uses constant divisors, immediates are exact bit
// patterns, and scalar inputs are loaded once per lane before the loop.

#include "minicompiler/fused_program.hpp"
#include "minicompiler/hip/hip_backend.hpp"
#include "minicompiler/tensor.hpp"

#include <cstddef>
#include <string>
#include <vector>

namespace minicompiler::hip {

inline constexpr const char* kElementwiseKernelName = "mc_elementwise";
// Lanes per block: four 64-wide waves. The generated kernel assumes it.
inline constexpr unsigned kElementwiseBlock = 256;
// Default cap of the elementwise grid, in blocks per CU.
inline constexpr int kElementwiseBlocksPerCu = 64;

struct CodegenOptions {
    // 16-byte accesses when every input allows them.
    bool allow_vectorize = true;
    // Vectors (or floats) each lane loads before it computes and stores: more
    // bytes in flight per wave to cover HBM latency. 0: by the program, 8
    // for programs of 8 or more ops (their arithmetic holds back each wave's
    // stores), else 4 (measured on an MI355X: GELU 4096^2 5.95 TB/s with 8
    // against 5.88 with 4; BatchNorm 6.19 with 4 against 6.10 with 8; copy
    // 6.28 with 4 against 6.08).
    unsigned items_per_lane = 0;
    // Non-temporal hints on the streaming loads and stores.
    bool nontemporal_loads = true;
    bool nontemporal_stores = true;
};

struct ElementwiseKernel {
    std::string source;
    bool vectorized = false;
    unsigned items_per_lane = 1;
    // Elements (or vectors) one block covers per step of its loop.
    unsigned items_per_block_step() const { return kElementwiseBlock * items_per_lane; }
};

// How the kernel reads one input of shape `in` for an output of shape `out`.
struct Access {
    enum class Kind {
        Contiguous,  // same element count as the output: element i
        Scalar,      // one element, loaded before the loop
        Periodic,    // a suffix of the output shape (a bias row): element i % period
        General,     // anything else: index expression with constant divisors
    };
    Kind kind = Kind::Contiguous;
    std::size_t period = 0;
    std::string index;  // General: expression in `i`
};

Access classify_access(const Shape& in, const Shape& out);

ElementwiseKernel generate_elementwise_kernel(const FusedProgram& program, const std::vector<Shape>& input_shapes,
                                              const Shape& out_shape, const CodegenOptions& options = {});

inline constexpr const char* kGemmEpilogueKernelName = "mc_gemm_epilogue";
inline constexpr const char* kSumSplitsEpilogueKernelName = "mc_sum_splits_epilogue";

struct GemmEpilogueKernel {
    std::string source;  // defines kGemmEpilogueKernelName (and, FP32, kSumSplitsEpilogueKernelName)
};

// Which GEMM body the epilogue kernel wraps.
enum class GemmBody {
    F32Mfma,      // fp32 operands, FP32 matrix cores, 128x128 tiles, 256 lanes, split K (gemm_f32_mfma.h)
    F32RingBig,   // the same arithmetic, LDS ring, persistent (gemm_f32_ring.h): 256x256 tiles, one block per CU
    F32RingWide,  // likewise, 128x128 tiles, 2 stages, up to two blocks per CU
    F32RingWide8,  // likewise, 128x128 tiles, one block of 8 waves per CU
    F32RingThin,  // likewise, 32x128 tiles (M <= 32, or when the autotuner picks it), 6 stages
    F32RingMid,   // likewise, 64x128 tiles, 3 stages, up to two blocks per CU (autotuner only)
    F32Narrow16,  // fp32 operands, 16x64 tiles on 16x16x4 MFMAs, K split over waves (gemm_f32_narrow.h), M <= 16
    F32Narrow32,  // likewise, 32x64 tiles (split_k products with at most one tile per CU)
    F32Narrow16x64,  // likewise, 16x64 tiles for M > 16 (short K, more tiles than 32x64 give)
    F32Narrow16x32,  // likewise, 16x32 tiles
    F32Narrow64,  // likewise, 64x64 tiles
    Bf16Fast,     // bf16 operands in HBM, 256x256 tiles, 512 lanes, one block per tile
    F16Fast,      // fp16 operands, likewise
};

inline bool is_narrow_body(GemmBody body) {
    return body == GemmBody::F32Narrow16 || body == GemmBody::F32Narrow32 || body == GemmBody::F32Narrow16x64 ||
           body == GemmBody::F32Narrow16x32 || body == GemmBody::F32Narrow64;
}

inline bool is_f32_body(GemmBody body) {
    return body == GemmBody::F32Mfma || body == GemmBody::F32RingBig || body == GemmBody::F32RingWide ||
           body == GemmBody::F32RingWide8 ||
           body == GemmBody::F32RingThin || body == GemmBody::F32RingMid || is_narrow_body(body);
}

// A narrow body's tile rows and columns, and its configuration's name in gemm_f32_narrow.h.
inline int narrow_rows(GemmBody body) {
    return body == GemmBody::F32Narrow64 ? 64 : body == GemmBody::F32Narrow32 ? 32 : 16;
}
inline int narrow_cols(GemmBody body) { return body == GemmBody::F32Narrow16x32 ? 32 : 64; }
inline const char* narrow_config(GemmBody body) {
    switch (body) {
        case GemmBody::F32Narrow16: return "McNarrow16";
        case GemmBody::F32Narrow16x64: return "McNarrow16x64";
        case GemmBody::F32Narrow16x32: return "McNarrow16x32";
        case GemmBody::F32Narrow64: return "McNarrow64";
        default: return "McNarrow32";
    }
}

// A GEMM (the matrix-core body in `gemm_body_source`, of kind `body`) whose
// store applies `program`, the
// fused elementwise group that consumes the GEMM's result: the program's
// input `acc_input` is the accumulated value; every other input is read at
// the flat output index by its access class against `out_shape`. Kernel
// arguments, FP32 bodies: (a, b, c, m, n, k, k_split, depth, partial,
// counters, epi) (two-stage: grid (N/128, M/128, depth) of 256 lanes; ring:
// the grid and block of mchip_f32_ring_plan) and, for split K, the sum
// kernel's (partial, c, count, depth, epi). With split K on a ring or narrow
// body and `counters` not null (one zeroed unsigned per tile), the GEMM
// launch adds the partials itself and the sum kernel is not launched; the
// two-stage body ignores counters. 16-bit bodies (one block of 512 lanes per
// 256x256 tile): (a, b, c, m, n, k, epi). epi holds one float pointer per program
// input (that of `acc_input` unused). `vectorized_operands` (FP32): A and B
// rows allow 16-byte loads (k and n multiples of 4, 16-byte aligned).
// The product's dimensions, when the kernel serves one shape only: the
// generated kernel then passes them to the body as constants (the index and
// address arithmetic folds, e.g. a bias read once per column instead of per
// element) and ignores its m, n, k, k_split and depth arguments.
struct GemmDims {
    int m = 0, n = 0, k = 0, k_split = 0, depth = 1;
};

GemmEpilogueKernel generate_gemm_epilogue_kernel(const FusedProgram& program, std::size_t acc_input,
                                                 const std::vector<Shape>& input_shapes, const Shape& out_shape,
                                                 bool vectorized_operands, const char* gemm_body_source,
                                                 GemmBody body = GemmBody::F32Mfma, const GemmDims& fixed = {});

// The generator options a compiled graph uses.
CodegenOptions codegen_options(const HipOptions& options);

// One unary or binary op as a program (load the operands, apply the op), so
// unfused graphs go through the same generator.
FusedProgram single_op_program(OpKind op);

}  // namespace minicompiler::hip
