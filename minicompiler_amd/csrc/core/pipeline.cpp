// Pass registry and runner (reference: src/passes/pipeline.cpp:8-74).

#include "minicompiler/passes/pipeline.hpp"

#include "minicompiler/passes/constant_folding.hpp"
#include "minicompiler/passes/dead_node_elimination.hpp"
#include "minicompiler/passes/operator_fusion.hpp"

namespace minicompiler {

namespace {

Result<Graph> run_fold(const Graph& g, PassReport* r) { return fold_constants(g, r); }

const PassInfo* lookup_pass(std::string_view name) {
    for (const PassInfo& p : registered_passes()) {
        if (name == p.name) return &p;
    }
    return nullptr;
}

std::string pass_names() {
    std::string s;
    for (const PassInfo& p : registered_passes()) s += (s.empty() ? "" : ", ") + std::string(p.name);
    return s;
}

}  // namespace

const std::vector<PassInfo>& registered_passes() {
    static const std::vector<PassInfo> passes = {
        {"dne", "dead-node elimination: remove nodes no output depends on", &eliminate_dead_nodes},
        {"fold", "constant folding: evaluate nodes whose operands are all constants", &run_fold},
        {"fuse", "operator fusion: merge groups of elementwise ops into single kernels", &fuse_elementwise},
    };
    return passes;
}

// Dead code first so nothing dead is folded; again after folding orphans
// operands; fuse; again to drop the scalars that became immediates.
const std::vector<std::string>& default_pipeline() {
    static const std::vector<std::string> p = {"dne", "fold", "dne", "fuse", "dne"};
    return p;
}

Result<std::vector<std::string>> parse_pipeline(std::string_view spec) {
    if (spec == "default") return default_pipeline();
    if (spec.empty() || spec == "none") return std::vector<std::string>{};
    std::vector<std::string> passes;
    std::size_t pos = 0;
    for (;;) {
        const std::size_t comma = spec.find(',', pos);
        const std::string_view name = spec.substr(pos, comma == std::string_view::npos ? std::string_view::npos : comma - pos);
        if (!lookup_pass(name)) return Error{"unknown pass '" + std::string(name) + "' (passes: " + pass_names() + ")"};
        passes.emplace_back(name);
        if (comma == std::string_view::npos) break;
        pos = comma + 1;
    }
    return passes;
}

Result<Graph> run_pipeline(const Graph& graph, const std::vector<std::string>& passes,
                           std::vector<PassReport>* reports, const PassObserver& observer) {
    Status st = graph.verify();
    if (!st.ok()) return Error{"input graph is invalid: " + st.message()};
    Graph current = graph;
    if (observer) observer(0, "input", current);
    for (std::size_t i = 0; i < passes.size(); ++i) {
        const PassInfo* pass = lookup_pass(passes[i]);
        if (!pass) return Error{"unknown pass '" + passes[i] + "'"};
        PassReport report;
        Result<Graph> next = pass->run(current, &report);
        if (!next.ok()) return Error{"pass '" + passes[i] + "' failed: " + next.error().message};
        st = next->verify();
        if (!st.ok()) return Error{"pass '" + passes[i] + "' produced an invalid graph: " + st.message()};
        current = std::move(next).value();
        if (reports) reports->push_back(std::move(report));
        if (observer) observer(i + 1, passes[i], current);
    }
    return current;
}

}  // namespace minicompiler
