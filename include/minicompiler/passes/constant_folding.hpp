#pragma once

// Replaces each compute node whose operands are all constants by a Constant
// holding its value (reference: include/minicompiler/passes/constant_folding.hpp:11-28).
// The values are computed on the host at compile time by
// fold_evaluate_node(), which follows the CPU backend's per-op float
// semantics; results above `max_elements` are left for run time.

#include "minicompiler/graph.hpp"
#include "minicompiler/passes/pass.hpp"
#include "minicompiler/result.hpp"

#include <cstddef>
#include <vector>

namespace minicompiler {

struct ConstantFoldingOptions {
    std::size_t max_elements = std::size_t{1} << 22;
};

Result<Graph> fold_constants(const Graph& graph, PassReport* report = nullptr,
                             const ConstantFoldingOptions& options = {});

// Compile-time evaluation of one compute node over host constants, operands
// in node order, every intermediate rounded to float.
void fold_evaluate_node(const Node& node, const std::vector<const float*>& operands,
                        const std::vector<Shape>& operand_shapes, float* out);

}  // namespace minicompiler
