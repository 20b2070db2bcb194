// The graph container (the contract of the reference's src/graph.cpp: nodes
// in a topological vector, typed by the ops, checked on insertion and by
// verify()).
//
// One admission check, vet(), serves both ways a node can be judged: the
// add_* calls build a Node and admit() it at the end of the vector, and
// verify() vets every stored node at its own position. A node is acceptable
// when its operands are earlier nodes, its operand count is its op's, its
// type can be stored, its payload (constant) or program (fused node) fits
// that type, and a primitive op's type is the one the op infers.

#include "minicompiler/graph.hpp"

#include <algorithm>

namespace minicompiler {

namespace {

// Why `t` cannot be the type of a stored tensor, or "" when it can.
std::string storage_problem(const TensorType& t) {
    if (t.dtype != DType::Float32) return "only f32 is supported, got " + to_string(t);
    if (std::any_of(t.shape.begin(), t.shape.end(), [](std::int64_t d) { return d < 1; })) {
        return "dimensions must be >= 1, got " + to_string(t);
    }
    if (!checked_num_elements(t.shape)) return to_string(t) + " has more than 2^31 - 1 elements";
    return {};
}

std::string describe(const Node& n, std::size_t position) {
    return "node %" + std::to_string(position) + " '" + n.name + "'";
}

}  // namespace

Status Graph::vet(const Node& n, std::size_t position) const {
    const std::string who = describe(n, position);
    for (NodeId in : n.inputs) {
        if (in < 0 || static_cast<std::size_t>(in) >= position) {
            return Error{who + ": operand %" + std::to_string(in) + " is not an earlier node"};
        }
    }
    const int arity = op_arity(n.op);
    if (arity >= 0 && static_cast<int>(n.inputs.size()) != arity) {
        return Error{who + ": " + op_name(n.op) + " takes " + std::to_string(arity) + " operand(s), got " +
                     std::to_string(n.inputs.size())};
    }
    const std::string bad_type = storage_problem(n.type);
    if (!bad_type.empty()) return Error{who + ": " + bad_type};

    std::vector<TensorType> operand_types;
    operand_types.reserve(n.inputs.size());
    for (NodeId in : n.inputs) operand_types.push_back(nodes_[static_cast<std::size_t>(in)].type);

    switch (n.op) {
        case OpKind::Input: return Status();
        case OpKind::Constant: {
            const std::size_t have = n.constant ? n.constant->size() : 0;
            if (have != n.type.num_elements()) {
                return Error{who + ": " + std::to_string(have) + " values given for " + to_string(n.type) + " (" +
                             std::to_string(n.type.num_elements()) + " needed)"};
            }
            return Status();
        }
        case OpKind::FusedElementwise: {
            if (!n.fused) return Error{who + ": fused node without a program"};
            Status st = validate(*n.fused, n.inputs.size());
            if (!st.ok()) return Error{who + ": " + st.message()};
            for (const TensorType& t : operand_types) {
                Result<Shape> b = broadcast_shapes(t.shape, n.type.shape);
                if (!b.ok() || b.value() != n.type.shape) {
                    return Error{who + ": operand " + to_string(t) + " does not broadcast to " + to_string(n.type)};
                }
            }
            return Status();
        }
        default: {
            Result<TensorType> t = infer_result_type(n.op, operand_types);
            if (!t.ok()) return Error{who + ": " + t.error().message};
            if (t.value() != n.type) {
                return Error{who + ": typed " + to_string(n.type) + " but " + op_name(n.op) + " gives " +
                             to_string(t.value())};
            }
            return Status();
        }
    }
}

Result<NodeId> Graph::admit(Node n) {
    const std::size_t position = nodes_.size();
    if (n.name.empty()) n.name = std::string(op_name(n.op)) + "_" + std::to_string(position);
    Status st = vet(n, position);
    if (!st.ok()) return st.error();
    const auto id = static_cast<NodeId>(position);
    if (n.op == OpKind::Input) inputs_.push_back(id);
    nodes_.push_back(std::move(n));
    return id;
}

Result<NodeId> Graph::add_input(std::string name, TensorType type) {
    Node n;
    n.op = OpKind::Input;
    n.name = std::move(name);
    n.type = std::move(type);
    return admit(std::move(n));
}

Result<NodeId> Graph::add_constant(std::string name, TensorType type, std::vector<float> values) {
    return add_constant(std::move(name), std::move(type),
                        std::make_shared<const std::vector<float>>(std::move(values)));
}

Result<NodeId> Graph::add_constant(std::string name, TensorType type,
                                   std::shared_ptr<const std::vector<float>> values) {
    Node n;
    n.op = OpKind::Constant;
    n.name = std::move(name);
    n.type = std::move(type);
    n.constant = std::move(values);
    return admit(std::move(n));
}

Result<NodeId> Graph::add_op(OpKind op, std::vector<NodeId> inputs, std::string name) {
    if (!is_elementwise(op) && op != OpKind::MatMul) {
        return Error{std::string("add_op makes elementwise and matmul nodes, not '") + op_name(op) + "'"};
    }
    // The result type comes from the operands, so they must exist first.
    const std::string label = name.empty() ? std::string(op_name(op)) : name;
    std::vector<TensorType> operand_types;
    for (NodeId in : inputs) {
        if (in < 0 || static_cast<std::size_t>(in) >= nodes_.size()) {
            return Error{label + ": operand %" + std::to_string(in) + " does not exist"};
        }
        operand_types.push_back(nodes_[static_cast<std::size_t>(in)].type);
    }
    Result<TensorType> type = infer_result_type(op, operand_types);
    if (!type.ok()) return Error{label + ": " + type.error().message};
    Node n;
    n.op = op;
    n.name = std::move(name);
    n.inputs = std::move(inputs);
    n.type = std::move(type).value();
    return admit(std::move(n));
}

Result<NodeId> Graph::add_fused(std::vector<NodeId> inputs, std::shared_ptr<const FusedProgram> program,
                                TensorType type, std::string name) {
    Node n;
    n.op = OpKind::FusedElementwise;
    n.name = std::move(name);
    n.inputs = std::move(inputs);
    n.type = std::move(type);
    n.fused = std::move(program);
    return admit(std::move(n));
}

Status Graph::add_output(NodeId id) {
    if (id < 0 || static_cast<std::size_t>(id) >= nodes_.size()) {
        return Error{"output %" + std::to_string(id) + " does not exist"};
    }
    if (is_output(id)) return Error{"'" + node(id).name + "' is already an output"};
    outputs_.push_back(id);
    return Status();
}

Result<NodeId> Graph::copy_node(const Node& prototype, std::vector<NodeId> inputs) {
    // Same kind, name, type and payload over the new operands; admit()
    // re-checks the type against the operands it now has.
    Node n = prototype;
    n.inputs = std::move(inputs);
    return admit(std::move(n));
}

bool Graph::is_output(NodeId id) const { return std::find(outputs_.begin(), outputs_.end(), id) != outputs_.end(); }

std::optional<NodeId> Graph::find(std::string_view name) const {
    const auto it = std::find_if(nodes_.begin(), nodes_.end(), [&](const Node& n) { return n.name == name; });
    if (it == nodes_.end()) return std::nullopt;
    return static_cast<NodeId>(it - nodes_.begin());
}

std::vector<std::vector<NodeId>> Graph::compute_users() const {
    std::vector<std::vector<NodeId>> users(nodes_.size());
    std::vector<NodeId> operands;
    for (std::size_t i = 0; i < nodes_.size(); ++i) {
        // A node reading one value twice (x * x) is one user of it.
        operands = nodes_[i].inputs;
        std::sort(operands.begin(), operands.end());
        operands.erase(std::unique(operands.begin(), operands.end()), operands.end());
        for (NodeId in : operands) users[static_cast<std::size_t>(in)].push_back(static_cast<NodeId>(i));
    }
    return users;
}

Status Graph::verify() const {
    for (std::size_t i = 0; i < nodes_.size(); ++i) {
        Status st = vet(nodes_[i], i);
        if (!st.ok()) return st;
    }
    // The input list names every input node exactly once and nothing else.
    std::vector<char> listed(nodes_.size(), 0);
    for (NodeId in : inputs_) {
        if (in < 0 || static_cast<std::size_t>(in) >= nodes_.size() || node(in).op != OpKind::Input) {
            return Error{"the input list names %" + std::to_string(in) + ", which is not an input node"};
        }
        if (listed[static_cast<std::size_t>(in)]++) return Error{"input '" + node(in).name + "' is listed twice"};
    }
    for (std::size_t i = 0; i < nodes_.size(); ++i) {
        if (nodes_[i].op == OpKind::Input && !listed[i]) {
            return Error{describe(nodes_[i], i) + ": an input node missing from the input list"};
        }
    }
    if (outputs_.empty()) return Error{"the graph has no outputs"};
    std::vector<char> output(nodes_.size(), 0);
    for (NodeId out : outputs_) {
        if (out < 0 || static_cast<std::size_t>(out) >= nodes_.size()) {
            return Error{"output %" + std::to_string(out) + " does not exist"};
        }
        if (output[static_cast<std::size_t>(out)]++) return Error{"'" + node(out).name + "' is an output twice"};
    }
    return Status();
}

GraphStats compute_stats(const Graph& graph) {
    GraphStats s;
    s.nodes = graph.num_nodes();
    for (const Node& n : graph.nodes()) {
        switch (n.op) {
            case OpKind::Input: ++s.inputs; continue;
            case OpKind::Constant: ++s.constants; continue;
            case OpKind::FusedElementwise:
                ++s.fused_nodes;
                s.elementwise_ops += n.fused->num_ops();
                break;
            case OpKind::MatMul: ++s.matmuls; break;
            default: ++s.elementwise_ops; break;
        }
        ++s.compute_nodes;
        ++s.op_counts[op_name(n.op)];
    }
    return s;
}

}  // namespace minicompiler
