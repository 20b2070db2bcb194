#pragma once

// Host tensors and seeded inputs (reference: include/minicompiler/runtime/host_tensor.hpp:13-25).

#include "minicompiler/graph.hpp"
#include "minicompiler/tensor.hpp"

#include <cstdint>
#include <utility>
#include <vector>

namespace minicompiler {

struct HostTensor {
    TensorType type;
    std::vector<float> data;

    HostTensor() = default;
    explicit HostTensor(TensorType t) : type(std::move(t)), data(type.num_elements()) {}
    HostTensor(TensorType t, std::vector<float> values) : type(std::move(t)), data(std::move(values)) {}
};

// Input k of `graph` filled with uniform_values(n, seed + k, lo, hi).
std::vector<HostTensor> make_random_inputs(const Graph& graph, std::uint64_t seed, float lo = -1.0f,
                                           float hi = 1.0f);

}  // namespace minicompiler
