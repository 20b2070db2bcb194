#pragma once

// The SSA DAG. Same surface as the reference's
// include/minicompiler/graph.hpp:24-109: nodes in a vector whose order is a
// topological order (operands must exist when a node is added), passes build
// new graphs, verify() re-checks every invariant.

#include "minicompiler/fused_program.hpp"
#include "minicompiler/ops.hpp"
#include "minicompiler/result.hpp"
#include "minicompiler/tensor.hpp"

#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <optional>
#include <string>
#include <string_view>
#include <vector>

namespace minicompiler {

using NodeId = std::int32_t;
inline constexpr NodeId kNoNode = -1;

struct Node {
    OpKind op = OpKind::Input;
    std::string name;
    std::vector<NodeId> inputs;
    TensorType type;
    // Constant payload, row-major; shared so copying a graph never copies weights.
    std::shared_ptr<const std::vector<float>> constant;
    // FusedElementwise body.
    std::shared_ptr<const FusedProgram> fused;
};

class Graph {
public:
    explicit Graph(std::string name = "graph") : name_(std::move(name)) {}

    const std::string& name() const { return name_; }

    // An empty name is replaced by "<op>_<id>".
    Result<NodeId> add_input(std::string name, TensorType type);
    Result<NodeId> add_constant(std::string name, TensorType type, std::vector<float> values);
    Result<NodeId> add_constant(std::string name, TensorType type, std::shared_ptr<const std::vector<float>> values);
    Result<NodeId> add_op(OpKind op, std::vector<NodeId> inputs, std::string name = {});
    Result<NodeId> add_fused(std::vector<NodeId> inputs, std::shared_ptr<const FusedProgram> program,
                             TensorType type, std::string name = {});
    Status add_output(NodeId id);

    // A node like `prototype` (kind, name, payload) over new operands.
    Result<NodeId> copy_node(const Node& prototype, std::vector<NodeId> inputs);

    std::size_t num_nodes() const { return nodes_.size(); }
    const Node& node(NodeId id) const { return nodes_[static_cast<std::size_t>(id)]; }
    const std::vector<Node>& nodes() const { return nodes_; }
    const std::vector<NodeId>& inputs() const { return inputs_; }
    const std::vector<NodeId>& outputs() const { return outputs_; }
    bool is_output(NodeId id) const;

    std::optional<NodeId> find(std::string_view name) const;

    // users[v]: distinct readers of v, ascending.
    std::vector<std::vector<NodeId>> compute_users() const;

    Status verify() const;

private:
    // Whether `n` may stand at index `position` of this graph: operands
    // earlier than it, the op's arity, a storable type, a payload or program
    // that fits it, and for primitive ops the type the op infers. Both the
    // add_* calls and verify() go through it.
    Status vet(const Node& n, std::size_t position) const;
    // vet(n) at the end of the graph, then store it (an unnamed node becomes
    // "<op>_<id>"; an input also joins the input list).
    Result<NodeId> admit(Node n);

    std::string name_;
    std::vector<Node> nodes_;
    std::vector<NodeId> inputs_;
    std::vector<NodeId> outputs_;
};

struct GraphStats {
    std::size_t nodes = 0;
    std::size_t inputs = 0;
    std::size_t constants = 0;
    std::size_t compute_nodes = 0;  // one kernel launch each on the GPU
    std::size_t fused_nodes = 0;
    std::size_t elementwise_ops = 0;  // primitive ops, including those inside fused nodes
    std::size_t matmuls = 0;
    std::map<std::string, std::size_t> op_counts;
};

GraphStats compute_stats(const Graph& graph);

}  // namespace minicompiler
