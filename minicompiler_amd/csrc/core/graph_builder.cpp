// Sticky-error builder (reference: src/graph_builder.cpp:5-54).

#include "minicompiler/graph_builder.hpp"

namespace minicompiler {

NodeId GraphBuilder::keep(Result<NodeId> r) {
    if (r.ok()) return r.value();
    first_error_ = r.error();
    return kNoNode;
}

NodeId GraphBuilder::input(std::string name, Shape shape) {
    if (first_error_) return kNoNode;
    return keep(graph_.add_input(std::move(name), TensorType(std::move(shape))));
}

NodeId GraphBuilder::constant(std::string name, Shape shape, std::vector<float> values) {
    if (first_error_) return kNoNode;
    return keep(graph_.add_constant(std::move(name), TensorType(std::move(shape)), std::move(values)));
}

NodeId GraphBuilder::scalar(std::string name, float value) { return constant(std::move(name), Shape{}, {value}); }

NodeId GraphBuilder::op(OpKind kind, std::vector<NodeId> inputs, std::string name) {
    if (first_error_) return kNoNode;
    return keep(graph_.add_op(kind, std::move(inputs), std::move(name)));
}

void GraphBuilder::output(NodeId id) {
    if (first_error_) return;
    Status st = graph_.add_output(id);
    if (!st.ok()) first_error_ = st.error();
}

Result<Graph> GraphBuilder::build() && {
    if (first_error_) return *first_error_;
    Status st = graph_.verify();
    if (!st.ok()) return st.error();
    return std::move(graph_);
}

}  // namespace minicompiler
