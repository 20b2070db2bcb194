#pragma once

// The .mcg text format. Same language as the reference's
// include/minicompiler/parser.hpp:12-38:
//
//   graph NAME                                  optional, before any node
//   dim B = 64                                  named dimension, overridable
//   input x : f32[B, 256]
//   const w : f32[256, 512] = uniform(seed=1, lo=-0.05, hi=0.05)
//   const b : f32[512] = 0.1                    every element 0.1
//   const v : f32[3] = [1, 2, 3]
//   h = matmul x, w
//   output y, z
//
// One addition: `normal(seed=S, mean=M, std=D)` initialises a constant from
// fill_normal (random.hpp), for the BatchNorm workload's statistics.

#include "minicompiler/graph.hpp"
#include "minicompiler/result.hpp"

#include <cstdint>
#include <map>
#include <string>
#include <string_view>

namespace minicompiler {

struct ParseOptions {
    std::map<std::string, std::int64_t> dims;  // overrides of `dim` defaults
};

Result<Graph> parse_graph(std::string_view text, const ParseOptions& options = {});
Result<Graph> parse_graph_file(const std::string& path, const ParseOptions& options = {});

// One line per node, as `mcc --print` shows it.
std::string print_graph(const Graph& graph);

// "0.5", "[1, 2, 3]" or "<4096 values>".
std::string describe_constant(const Node& constant);

}  // namespace minicompiler
