#pragma once

// Text of the kernel headers the library compiles at run time with
// generated code (the build embeds them; see EMBEDDED in build.py).

namespace minicompiler::hip {

// gemm_f32_mfma.h: the FP32 matrix-core GEMM body with an epilogue hook.
extern const char* const kGemmF32MfmaSource;
// gemm_f32_ring.h: the FP32 matrix-core GEMM body with an LDS ring and
// persistent blocks, with an epilogue hook (the same arithmetic).
extern const char* const kGemmF32RingSource;
// gemm_f32_narrow.h: the FP32 narrow-tile GEMM body (16x16x4 MFMAs, no
// LDS staging) with an epilogue hook.
extern const char* const kGemmF32NarrowSource;
// gemm_split_arrival.h: the split-K arrival count the ring and narrow bodies
// use to add K splits in the GEMM launch (goes before them).
extern const char* const kGemmSplitArrivalSource;
// gemm_mfma16_fast.h: the bf16 / fp16 matrix-core GEMM body (16-bit inputs
// in HBM) with an epilogue hook.
extern const char* const kGemm16FastSource;

}  // namespace minicompiler::hip
