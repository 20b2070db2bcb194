#pragma once

// Removes every node no graph output depends on; graph inputs always stay
// (reference: include/minicompiler/passes/dead_node_elimination.hpp:11-19).

#include "minicompiler/graph.hpp"
#include "minicompiler/passes/pass.hpp"
#include "minicompiler/result.hpp"

namespace minicompiler {

Result<Graph> eliminate_dead_nodes(const Graph& graph, PassReport* report = nullptr);

}  // namespace minicompiler
