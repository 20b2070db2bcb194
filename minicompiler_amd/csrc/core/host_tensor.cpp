// Seeded graph inputs (reference: src/runtime/host_tensor.cpp:7-14).

#include "minicompiler/runtime/host_tensor.hpp"

#include "minicompiler/random.hpp"

namespace minicompiler {

std::vector<HostTensor> make_random_inputs(const Graph& graph, std::uint64_t seed, float lo, float hi) {
    std::vector<HostTensor> inputs;
    inputs.reserve(graph.inputs().size());
    std::uint64_t s = seed;
    for (NodeId id : graph.inputs()) {
        const TensorType& t = graph.node(id).type;
        inputs.emplace_back(t, uniform_values(t.num_elements(), s++, lo, hi));
    }
    return inputs;
}

}  // namespace minicompiler
