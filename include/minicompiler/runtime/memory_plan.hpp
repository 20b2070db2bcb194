#pragma once

// Lifetime-based buffer reuse (reference: include/minicompiler/runtime/memory_plan.hpp:11-45).
//
// Nodes run in id order, so an id is a time step. A compute node's value gets
// a free buffer (the smallest that fits; else the largest free one, grown;
// else a new one) before its operands' buffers are released, so no node
// writes a buffer it still reads. A value nothing reads is released at once.
// Inputs and constants are never pooled. The HIP backend lays the buffers
// out as offsets of one device arena.

#include "minicompiler/graph.hpp"

#include <cstddef>
#include <cstdint>
#include <vector>

namespace minicompiler {

struct PlanOptions {
    // Give graph outputs pooled buffers (false: the caller's memory holds them).
    bool pool_outputs = true;
};

struct MemoryPlan {
    static constexpr std::int32_t kNotPooled = -1;

    std::vector<std::int32_t> buffer_of;    // per node
    std::vector<std::size_t> buffer_bytes;  // per buffer
    std::vector<NodeId> last_use;           // per node; num_nodes() for outputs, kNoNode if unread

    std::size_t bytes_without_reuse = 0;
    std::size_t bytes_with_reuse() const;
};

MemoryPlan plan_memory(const Graph& graph, const PlanOptions& options = {});

}  // namespace minicompiler
