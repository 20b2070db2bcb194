#pragma once

// Elementwise fusion (reference: include/minicompiler/passes/operator_fusion.hpp:12-44).
//
// A group grows from a root (visited from the last node down) toward its
// producers; a producer joins when it is elementwise, has the root's shape,
// is not a graph output, and every one of its users is already in the group
// (which keeps groups convex). Groups of two or more nodes are returned in
// topological order of their roots, members ascending.

#include "minicompiler/graph.hpp"
#include "minicompiler/passes/pass.hpp"
#include "minicompiler/result.hpp"

#include <vector>

namespace minicompiler {

std::vector<std::vector<NodeId>> find_fusion_groups(const Graph& graph);

// Each group becomes one FusedElementwise node at its root's position, named
// after the root; each distinct external operand is loaded once and scalar
// constants become immediates.
Result<Graph> fuse_elementwise(const Graph& graph, PassReport* report = nullptr);

}  // namespace minicompiler
