#pragma once

// What one pass did (reference: include/minicompiler/passes/pass.hpp:10-24).

#include "minicompiler/graph.hpp"

#include <string>

namespace minicompiler {

struct PassReport {
    std::string pass;
    GraphStats before;
    GraphStats after;
    std::string summary;
};

inline void fill_report(PassReport* report, const char* pass, const Graph& before, const Graph& after,
                        std::string summary) {
    if (report == nullptr) return;
    report->pass = pass;
    report->before = compute_stats(before);
    report->after = compute_stats(after);
    report->summary = std::move(summary);
}

}  // namespace minicompiler
