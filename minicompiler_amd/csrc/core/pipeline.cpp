// Pass registry and pipeline runner (the contract of the reference's
// src/passes/pipeline.cpp: three passes by name, the default order
// dne, fold, dne, fuse, dne, the graph verified before the first pass and
// after every pass, one report per pass).

#include "minicompiler/passes/pipeline.hpp"

#include "minicompiler/passes/constant_folding.hpp"
#include "minicompiler/passes/dead_node_elimination.hpp"
#include "minicompiler/passes/operator_fusion.hpp"

namespace minicompiler {

namespace {

Result<Graph> fold_pass(const Graph& g, PassReport* r) { return fold_constants(g, r); }

const PassInfo* pass_named(std::string_view name) {
    for (const PassInfo& p : registered_passes()) {
        if (name == p.name) return &p;
    }
    return nullptr;
}

// "a,b,,c" -> {"a", "b", "", "c"}.
std::vector<std::string_view> comma_items(std::string_view spec) {
    std::vector<std::string_view> items;
    for (;;) {
        const std::size_t comma = spec.find(',');
        items.push_back(spec.substr(0, comma));
        if (comma == std::string_view::npos) return items;
        spec.remove_prefix(comma + 1);
    }
}

}  // namespace

const std::vector<PassInfo>& registered_passes() {
    static const std::vector<PassInfo> passes = {
        {"dne", "drop every node that no graph output reads, directly or through others", &eliminate_dead_nodes},
        {"fold", "replace nodes computable from constants alone by their values", &fold_pass},
        {"fuse", "merge connected same-shape elementwise ops into one generated kernel each", &fuse_elementwise},
    };
    return passes;
}

// Dead nodes go first so nothing dead is folded; folding orphans the
// operands it consumed; fusion turns scalar constants into immediates, which
// orphans those constants.
const std::vector<std::string>& default_pipeline() {
    static const std::vector<std::string> order = {"dne", "fold", "dne", "fuse", "dne"};
    return order;
}

Result<std::vector<std::string>> parse_pipeline(std::string_view spec) {
    if (spec == "default") return default_pipeline();
    std::vector<std::string> passes;
    if (spec.empty() || spec == "none") return passes;
    for (std::string_view item : comma_items(spec)) {
        if (pass_named(item) == nullptr) {
            std::string known;
            for (const PassInfo& p : registered_passes()) known += (known.empty() ? "" : ", ") + std::string(p.name);
            return Error{"unknown pass '" + std::string(item) + "' (passes: " + known + ")"};
        }
        passes.emplace_back(item);
    }
    return passes;
}

Result<Graph> run_pipeline(const Graph& graph, const std::vector<std::string>& passes,
                           std::vector<PassReport>* reports, const PassObserver& observer) {
    if (Status st = graph.verify(); !st.ok()) return Error{"the graph is invalid before any pass: " + st.message()};
    Graph current = graph;
    if (observer) observer(0, "input", current);
    std::size_t stage = 0;
    for (const std::string& name : passes) {
        const PassInfo* pass = pass_named(name);
        if (pass == nullptr) return Error{"unknown pass '" + name + "'"};
        PassReport report;
        Result<Graph> next = pass->run(current, &report);
        if (!next.ok()) return Error{"pass '" + name + "': " + next.error().message};
        if (Status st = next->verify(); !st.ok()) {
            return Error{"pass '" + name + "' left an invalid graph: " + st.message()};
        }
        current = std::move(next).value();
        ++stage;
        if (reports) reports->push_back(std::move(report));
        if (observer) observer(stage, name, current);
    }
    return current;
}

}  // namespace minicompiler
