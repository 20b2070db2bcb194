// Dead-node elimination (the contract of the reference's
// src/passes/dead_node_elimination.cpp: keep what the outputs read, directly
// or transitively, and every graph input; renumber the rest in order).
//
// Reachability is a depth-first walk over operand edges from the outputs
// with an explicit stack; the kept nodes are then copied in their old order,
// which stays topological.

#include "minicompiler/passes/dead_node_elimination.hpp"

#include <vector>

namespace minicompiler {

namespace {

std::vector<char> needed_by_outputs(const Graph& graph) {
    std::vector<char> keep(graph.num_nodes(), 0);
    std::vector<NodeId> stack(graph.outputs().begin(), graph.outputs().end());
    while (!stack.empty()) {
        const NodeId id = stack.back();
        stack.pop_back();
        char& k = keep[static_cast<std::size_t>(id)];
        if (k) continue;
        k = 1;
        for (NodeId in : graph.node(id).inputs) {
            if (!keep[static_cast<std::size_t>(in)]) stack.push_back(in);
        }
    }
    // The inputs are the graph's calling convention: an unread one stays.
    for (NodeId in : graph.inputs()) keep[static_cast<std::size_t>(in)] = 1;
    return keep;
}

}  // namespace

Result<Graph> eliminate_dead_nodes(const Graph& graph, PassReport* report) {
    const std::vector<char> keep = needed_by_outputs(graph);
    Graph kept(graph.name());
    std::vector<NodeId> renumbered(graph.num_nodes(), kNoNode);
    std::size_t dropped = 0;
    for (std::size_t i = 0; i < graph.num_nodes(); ++i) {
        if (!keep[i]) {
            ++dropped;
            continue;
        }
        const Node& n = graph.node(static_cast<NodeId>(i));
        std::vector<NodeId> operands(n.inputs.size());
        for (std::size_t j = 0; j < n.inputs.size(); ++j) operands[j] = renumbered[static_cast<std::size_t>(n.inputs[j])];
        Result<NodeId> id = kept.copy_node(n, std::move(operands));
        if (!id.ok()) return id.error();
        renumbered[i] = id.value();
    }
    for (NodeId out : graph.outputs()) {
        if (Status st = kept.add_output(renumbered[static_cast<std::size_t>(out)]); !st.ok()) return st.error();
    }
    fill_report(report, "dne", graph, kept, "removed " + std::to_string(dropped) + " dead node(s)");
    return kept;
}

}  // namespace minicompiler
