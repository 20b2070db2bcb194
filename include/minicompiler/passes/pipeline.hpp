#pragma once

// Pass registry and pipeline runner (reference:
// include/minicompiler/passes/pipeline.hpp:15-41). The default pipeline is
// dne, fold, dne, fuse, dne; the graph is verified before the first pass and
// after each one.

#include "minicompiler/graph.hpp"
#include "minicompiler/passes/pass.hpp"
#include "minicompiler/result.hpp"

#include <cstddef>
#include <functional>
#include <string>
#include <string_view>
#include <vector>

namespace minicompiler {

using PassFn = Result<Graph> (*)(const Graph&, PassReport*);

struct PassInfo {
    const char* name;
    const char* description;
    PassFn run;
};

const std::vector<PassInfo>& registered_passes();
const std::vector<std::string>& default_pipeline();

// "default", "none" (or empty), or a comma-separated list of pass names.
Result<std::vector<std::string>> parse_pipeline(std::string_view spec);

using PassObserver = std::function<void(std::size_t stage, const std::string& pass, const Graph& graph)>;

Result<Graph> run_pipeline(const Graph& graph, const std::vector<std::string>& passes,
                           std::vector<PassReport>* reports = nullptr, const PassObserver& observer = {});

}  // namespace minicompiler
