// Backend registry (reference: src/runtime/backend.cpp:11-32). This library
// carries one backend, "hip". The reference's "cpu" backend is its Eigen
// implementation; it is not part of this library.

#include "minicompiler/runtime/backend.hpp"

#include "minicompiler/hip/hip_backend.hpp"

namespace minicompiler {

std::vector<std::string> available_backends() { return {"hip"}; }

Result<std::unique_ptr<Backend>> create_backend(std::string_view name) {
    if (name == "hip") return hip::make_hip_backend();
    std::string known;
    for (const std::string& b : available_backends()) known += (known.empty() ? "" : ", ") + b;
    if (name == "cpu" || name == "cuda") {
        return Error{"backend '" + std::string(name) + "' is not built into this library (available: " + known + ")"};
    }
    return Error{"unknown backend '" + std::string(name) + "' (available: " + known + ")"};
}

}  // namespace minicompiler
