// Dead-node elimination by mark and sweep (reference:
// src/passes/dead_node_elimination.cpp:7-42). A node's users come after it,
// so one walk from the last node down marks everything the outputs need.

#include "minicompiler/passes/dead_node_elimination.hpp"

#include <vector>

namespace minicompiler {

Result<Graph> eliminate_dead_nodes(const Graph& graph, PassReport* report) {
    const std::size_t n = graph.num_nodes();
    std::vector<char> live(n, 0);
    for (NodeId out : graph.outputs()) live[static_cast<std::size_t>(out)] = 1;
    for (std::size_t i = n; i-- > 0;) {
        if (!live[i]) continue;
        for (NodeId in : graph.node(static_cast<NodeId>(i)).inputs) live[static_cast<std::size_t>(in)] = 1;
    }
    // Inputs are the graph's calling convention: never removed.
    for (NodeId in : graph.inputs()) live[static_cast<std::size_t>(in)] = 1;

    Graph result(graph.name());
    std::vector<NodeId> new_id(n, kNoNode);
    std::size_t removed = 0;
    for (std::size_t i = 0; i < n; ++i) {
        if (!live[i]) {
            ++removed;
            continue;
        }
        const Node& node = graph.node(static_cast<NodeId>(i));
        std::vector<NodeId> operands;
        operands.reserve(node.inputs.size());
        for (NodeId in : node.inputs) operands.push_back(new_id[static_cast<std::size_t>(in)]);
        Result<NodeId> id = result.copy_node(node, std::move(operands));
        if (!id.ok()) return id.error();
        new_id[i] = id.value();
    }
    for (NodeId out : graph.outputs()) {
        Status st = result.add_output(new_id[static_cast<std::size_t>(out)]);
        if (!st.ok()) return st.error();
    }
    fill_report(report, "dne", graph, result, "removed " + std::to_string(removed) + " dead node(s)");
    return result;
}

}  // namespace minicompiler
