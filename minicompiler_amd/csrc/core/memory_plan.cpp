// Lifetime-based buffer planner (reference: src/runtime/memory_plan.cpp:12-70).
// The assignment rule is the reference's, step for step, because buffer
// counts and reuse are part of the compiled contract (tests pin them):
// best fit among free buffers, else grow the largest free buffer, else open
// a new one; a node's operands are released only after its own buffer is
// chosen; an unread value releases its buffer at once.

#include "minicompiler/runtime/memory_plan.hpp"

#include <algorithm>
#include <numeric>

namespace minicompiler {

std::size_t MemoryPlan::bytes_with_reuse() const {
    return std::accumulate(buffer_bytes.begin(), buffer_bytes.end(), std::size_t{0});
}

MemoryPlan plan_memory(const Graph& graph, const PlanOptions& options) {
    const std::size_t n = graph.num_nodes();
    MemoryPlan plan;
    plan.buffer_of.assign(n, MemoryPlan::kNotPooled);
    plan.last_use.assign(n, kNoNode);
    for (std::size_t i = 0; i < n; ++i) {
        for (NodeId in : graph.node(static_cast<NodeId>(i)).inputs) {
            plan.last_use[static_cast<std::size_t>(in)] = static_cast<NodeId>(i);
        }
    }
    for (NodeId out : graph.outputs()) plan.last_use[static_cast<std::size_t>(out)] = static_cast<NodeId>(n);

    std::vector<std::int32_t> free_list;
    for (std::size_t i = 0; i < n; ++i) {
        const auto id = static_cast<NodeId>(i);
        const Node& node = graph.node(id);
        if (!is_compute(node.op)) continue;
        const bool pooled = options.pool_outputs || !graph.is_output(id);
        if (pooled) {
            const std::size_t need = node.type.size_bytes();
            plan.bytes_without_reuse += need;
            auto pick = free_list.end();
            for (auto it = free_list.begin(); it != free_list.end(); ++it) {
                const std::size_t have = plan.buffer_bytes[static_cast<std::size_t>(*it)];
                if (have >= need && (pick == free_list.end() || have < plan.buffer_bytes[static_cast<std::size_t>(*pick)])) {
                    pick = it;
                }
            }
            if (pick == free_list.end() && !free_list.empty()) {
                pick = std::max_element(free_list.begin(), free_list.end(), [&](std::int32_t a, std::int32_t b) {
                    return plan.buffer_bytes[static_cast<std::size_t>(a)] < plan.buffer_bytes[static_cast<std::size_t>(b)];
                });
                plan.buffer_bytes[static_cast<std::size_t>(*pick)] = need;
            }
            if (pick != free_list.end()) {
                plan.buffer_of[i] = *pick;
                free_list.erase(pick);
            } else {
                plan.buffer_of[i] = static_cast<std::int32_t>(plan.buffer_bytes.size());
                plan.buffer_bytes.push_back(need);
            }
        }
        // Release operands whose last reader is this node (once per distinct
        // operand), also when this node's own value is not pooled.
        for (std::size_t k = 0; k < node.inputs.size(); ++k) {
            const NodeId in = node.inputs[k];
            const bool seen = std::find(node.inputs.begin(), node.inputs.begin() + static_cast<std::ptrdiff_t>(k), in) !=
                              node.inputs.begin() + static_cast<std::ptrdiff_t>(k);
            const auto ii = static_cast<std::size_t>(in);
            if (!seen && plan.buffer_of[ii] != MemoryPlan::kNotPooled && plan.last_use[ii] == id) {
                free_list.push_back(plan.buffer_of[ii]);
            }
        }
        if (pooled && plan.last_use[i] == kNoNode) free_list.push_back(plan.buffer_of[i]);
    }
    return plan;
}

}  // namespace minicompiler
