#pragma once

// hipRTC compilation of generated kernels with a process-wide cache
// (replaces the reference's src/cuda/kernel_compiler.hpp:15-36, which used
// NVRTC and the CUDA driver). Each distinct (architecture, options, source)
// is compiled once per process; a hit costs one map lookup. When the
// environment variable MINICOMPILER_HIP_CACHE_DIR names a directory, code
// objects are also kept there across processes. Thread-safe.

#include "minicompiler/result.hpp"

#include <map>
#include <mutex>
#include <string>
#include <vector>

namespace minicompiler::hip {

struct CompiledKernel {
    void* module = nullptr;
    void* function = nullptr;
};

class KernelCompiler {
public:
    static KernelCompiler& instance();

    // The hipRTC options every generated kernel is built with: the target,
    // -O3, no FP contraction (each op rounds to float), no packed FP32.
    static std::vector<std::string> options_for(const std::string& arch);

    // Function `name` of `source` compiled for `arch` (e.g. "gfx950") and
    // loaded on `device`, which must be the calling thread's current device
    // (modules are per device). `compile_ms` receives the hipRTC time
    // (0 on a cache hit). Errors carry the compiler log and the source.
    Result<CompiledKernel> get(const std::string& source, const char* name, const std::string& arch, int device,
                               double* compile_ms = nullptr);

    // Compiles to a code object only (no device needed).
    static Result<std::string> compile_code_object(const std::string& source, const std::string& arch,
                                                   double* compile_ms = nullptr);

private:
    std::mutex mutex_;
    std::map<std::string, CompiledKernel> loaded_;   // (device, arch, options, source, name) -> function
    std::map<std::string, void*> modules_;           // (device, arch, options, source) -> module
};

}  // namespace minicompiler::hip
