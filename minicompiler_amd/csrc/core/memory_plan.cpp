// Lifetime-based buffer planning (the contract of the reference's
// src/runtime/memory_plan.cpp: its buffer counts and sizes are pinned by the
// reference's tests).
//
// Node ids are time steps. Each pooled value lives from its own step to its
// last reader's (outputs to the end of the run; an unread value only for its
// own step). The planner walks the steps keeping the free buffers in a pool
// ordered by size:
//   1. the step's value takes the smallest free buffer that holds it; if none
//      does, the largest free buffer, grown to its size; if the pool is
//      empty, a new buffer;
//   2. then the values whose lifetime ends at this step return their buffers
//      to the pool (so a node never writes a buffer it still reads), and so
//      does the step's own value when nothing reads it.
// Among free buffers of one size the one returned first is taken first. The
// counts and sizes do not depend on that choice: buffers of one size are
// interchangeable for every later step.

#include "minicompiler/runtime/memory_plan.hpp"

#include <map>
#include <numeric>

namespace minicompiler {

std::size_t MemoryPlan::bytes_with_reuse() const {
    return std::accumulate(buffer_bytes.begin(), buffer_bytes.end(), std::size_t{0});
}

MemoryPlan plan_memory(const Graph& graph, const PlanOptions& options) {
    const std::size_t steps = graph.num_nodes();
    MemoryPlan plan;
    plan.buffer_of.assign(steps, MemoryPlan::kNotPooled);
    plan.last_use.assign(steps, kNoNode);
    for (std::size_t t = 0; t < steps; ++t) {
        for (NodeId in : graph.node(static_cast<NodeId>(t)).inputs) {
            plan.last_use[static_cast<std::size_t>(in)] = static_cast<NodeId>(t);
        }
    }
    for (NodeId out : graph.outputs()) plan.last_use[static_cast<std::size_t>(out)] = static_cast<NodeId>(steps);

    auto pooled = [&](std::size_t v) {
        const NodeId id = static_cast<NodeId>(v);
        return is_compute(graph.node(id).op) && (options.pool_outputs || !graph.is_output(id));
    };
    // ends_at[t]: pooled values whose last reader is step t, in id order.
    std::vector<std::vector<std::size_t>> ends_at(steps);
    for (std::size_t v = 0; v < steps; ++v) {
        const NodeId last = plan.last_use[v];
        if (pooled(v) && last != kNoNode && static_cast<std::size_t>(last) < steps) {
            ends_at[static_cast<std::size_t>(last)].push_back(v);
        }
    }

    std::multimap<std::size_t, std::int32_t> pool;  // free buffers by size, in the order returned
    auto give_back = [&](std::int32_t buffer) {
        pool.emplace(plan.buffer_bytes[static_cast<std::size_t>(buffer)], buffer);
    };
    auto take = [&](std::size_t bytes) -> std::int32_t {
        auto fit = pool.lower_bound(bytes);
        if (fit == pool.end() && !pool.empty()) {
            fit = pool.lower_bound(pool.rbegin()->first);  // the first returned of the largest
            plan.buffer_bytes[static_cast<std::size_t>(fit->second)] = bytes;
        }
        if (fit == pool.end()) {
            plan.buffer_bytes.push_back(bytes);
            return static_cast<std::int32_t>(plan.buffer_bytes.size() - 1);
        }
        const std::int32_t buffer = fit->second;
        pool.erase(fit);
        return buffer;
    };

    for (std::size_t t = 0; t < steps; ++t) {
        if (!is_compute(graph.node(static_cast<NodeId>(t)).op)) continue;
        const bool own = pooled(t);
        if (own) {
            const std::size_t bytes = graph.node(static_cast<NodeId>(t)).type.size_bytes();
            plan.bytes_without_reuse += bytes;
            plan.buffer_of[t] = take(bytes);
        }
        for (std::size_t v : ends_at[t]) give_back(plan.buffer_of[v]);
        if (own && plan.last_use[t] == kNoNode) give_back(plan.buffer_of[t]);
    }
    return plan;
}

}  // namespace minicompiler
