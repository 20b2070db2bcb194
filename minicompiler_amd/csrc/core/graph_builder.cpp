// The graph builder with a sticky error (the contract of the reference's
// src/graph_builder.cpp): once a call fails, every later call is a no-op
// returning kNoNode, and build() reports the first failure.

#include "minicompiler/graph_builder.hpp"

namespace minicompiler {

namespace {

// Runs `add` unless an earlier call failed; a failure is remembered.
template <typename Add>
NodeId guarded(std::optional<Error>& first_error, Add&& add) {
    if (first_error) return kNoNode;
    Result<NodeId> r = add();
    if (!r.ok()) {
        first_error = r.error();
        return kNoNode;
    }
    return r.value();
}

}  // namespace

NodeId GraphBuilder::input(std::string name, Shape shape) {
    return guarded(first_error_, [&] { return graph_.add_input(std::move(name), TensorType(std::move(shape))); });
}

NodeId GraphBuilder::constant(std::string name, Shape shape, std::vector<float> values) {
    return guarded(first_error_, [&] {
        return graph_.add_constant(std::move(name), TensorType(std::move(shape)), std::move(values));
    });
}

NodeId GraphBuilder::scalar(std::string name, float value) {
    return constant(std::move(name), Shape{}, std::vector<float>{value});
}

NodeId GraphBuilder::op(OpKind kind, std::vector<NodeId> inputs, std::string name) {
    return guarded(first_error_, [&] { return graph_.add_op(kind, std::move(inputs), std::move(name)); });
}

void GraphBuilder::output(NodeId id) {
    guarded(first_error_, [&]() -> Result<NodeId> {
        Status st = graph_.add_output(id);
        if (!st.ok()) return st.error();
        return id;
    });
}

Result<Graph> GraphBuilder::build() && {
    if (first_error_) return *first_error_;
    if (Status st = graph_.verify(); !st.ok()) return st.error();
    return std::move(graph_);
}

}  // namespace minicompiler
