#pragma once

// The backend plugin interface (reference: include/minicompiler/runtime/backend.hpp:18-49).
// This library registers one backend, "hip". Executables are not thread-safe:
// their buffers are allocated once and reused by every run.

#include "minicompiler/graph.hpp"
#include "minicompiler/result.hpp"
#include "minicompiler/runtime/host_tensor.hpp"

#include <cstddef>
#include <memory>
#include <string>
#include <string_view>
#include <vector>

namespace minicompiler {

class Executable {
public:
    virtual ~Executable() = default;

    // `inputs` follow Graph::inputs() in order and type; `outputs` is resized
    // to Graph::outputs() (its storage is reused by later runs) and must be a
    // different vector.
    virtual Status run(const std::vector<HostTensor>& inputs, std::vector<HostTensor>& outputs) = 0;

    // Caller-owned host memory; an output may not overlap an input.
    virtual Status run_buffers(const std::vector<const float*>& inputs, const std::vector<float*>& outputs) = 0;

    // Bytes of pooled intermediate storage after reuse.
    virtual std::size_t intermediate_bytes() const = 0;
};

class Backend {
public:
    virtual ~Backend() = default;
    virtual const char* name() const = 0;
    virtual Result<std::unique_ptr<Executable>> compile(const Graph& graph) = 0;
};

std::vector<std::string> available_backends();
Result<std::unique_ptr<Backend>> create_backend(std::string_view name);

}  // namespace minicompiler
