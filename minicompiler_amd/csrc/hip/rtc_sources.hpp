#pragma once

// Text of the kernel headers the library compiles at run time with
// generated code (the build embeds them; see EMBEDDED in build.py).

namespace minicompiler::hip {

// gemm_f32_mfma.h: the FP32 matrix-core GEMM body with an epilogue hook.
extern const char* const kGemmF32MfmaSource;

}  // namespace minicompiler::hip
