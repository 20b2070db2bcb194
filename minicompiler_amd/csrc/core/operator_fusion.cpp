// Elementwise fusion (reference: src/passes/operator_fusion.cpp:10-144).
// Group growth and instruction order follow the reference exactly, since
// stage counts and programs are part of the compiled contract: roots are
// visited from the highest id down, candidate producers are taken highest id
// first, members are emitted in ascending id order, and within a member the
// first operand's load or immediate is emitted before the second's.

#include "minicompiler/passes/operator_fusion.hpp"

#include <algorithm>
#include <map>
#include <memory>
#include <queue>

namespace minicompiler {

std::vector<std::vector<NodeId>> find_fusion_groups(const Graph& graph) {
    const std::size_t n = graph.num_nodes();
    const auto users = graph.compute_users();
    std::vector<int> group(n, -1);
    std::vector<std::vector<NodeId>> found;

    for (std::size_t i = n; i-- > 0;) {
        const Node& root = graph.node(static_cast<NodeId>(i));
        if (!is_elementwise(root.op) || group[i] >= 0) continue;
        const int g = static_cast<int>(found.size());
        group[i] = g;
        std::vector<NodeId> members{static_cast<NodeId>(i)};
        std::priority_queue<NodeId> frontier;
        for (NodeId in : root.inputs) frontier.push(in);
        while (!frontier.empty()) {
            const NodeId p = frontier.top();
            frontier.pop();
            const auto pi = static_cast<std::size_t>(p);
            if (group[pi] >= 0) continue;
            const Node& pn = graph.node(p);
            if (!is_elementwise(pn.op) || pn.type.shape != root.type.shape || graph.is_output(p)) continue;
            // Every reader of p must already be inside: p's value never
            // leaves the kernel, and the group stays convex.
            const bool contained =
                std::all_of(users[pi].begin(), users[pi].end(), [&](NodeId u) { return group[u] == g; });
            if (!contained) continue;
            group[pi] = g;
            members.push_back(p);
            for (NodeId in : pn.inputs) frontier.push(in);
        }
        std::sort(members.begin(), members.end());
        found.push_back(std::move(members));
    }

    // Roots were visited last-first; report them first-last.
    std::vector<std::vector<NodeId>> groups;
    for (auto it = found.rbegin(); it != found.rend(); ++it) {
        if (it->size() >= 2) groups.push_back(std::move(*it));
    }
    return groups;
}

namespace {

// Builds one group's FusedProgram over its external operands.
class ProgramEmitter {
public:
    ProgramEmitter(const Graph& graph, const std::vector<NodeId>& new_id) : graph_(graph), new_id_(new_id) {}

    void member(NodeId id) {
        const Node& node = graph_.node(id);
        const std::int32_t x = reg(node.inputs[0]);
        if (is_unary_elementwise(node.op)) {
            push(id, FusedInstr::unary(node.op, x));
        } else {
            const std::int32_t y = reg(node.inputs[1]);
            push(id, FusedInstr::binary(node.op, x, y));
        }
        program_->source_nodes.push_back(node.name);
    }

    std::shared_ptr<FusedProgram> program() const { return program_; }
    const std::vector<NodeId>& externals() const { return externals_; }

private:
    // The register holding node `id`, created on first use for an external
    // operand: an immediate for a one-element constant, else a load.
    std::int32_t reg(NodeId id) {
        const auto it = reg_.find(id);
        if (it != reg_.end()) return it->second;
        const Node& node = graph_.node(id);
        if (node.op == OpKind::Constant && node.type.num_elements() == 1) {
            return push(id, FusedInstr::imm((*node.constant)[0]));
        }
        externals_.push_back(new_id_[static_cast<std::size_t>(id)]);
        return push(id, FusedInstr::load(static_cast<std::int32_t>(externals_.size()) - 1));
    }

    std::int32_t push(NodeId id, FusedInstr ins) {
        program_->instrs.push_back(ins);
        const auto r = static_cast<std::int32_t>(program_->instrs.size()) - 1;
        reg_[id] = r;
        return r;
    }

    const Graph& graph_;
    const std::vector<NodeId>& new_id_;
    std::shared_ptr<FusedProgram> program_ = std::make_shared<FusedProgram>();
    std::vector<NodeId> externals_;
    std::map<NodeId, std::int32_t> reg_;
};

}  // namespace

Result<Graph> fuse_elementwise(const Graph& graph, PassReport* report) {
    const auto groups = find_fusion_groups(graph);
    std::vector<int> group_of(graph.num_nodes(), -1);
    for (std::size_t g = 0; g < groups.size(); ++g) {
        for (NodeId m : groups[g]) group_of[static_cast<std::size_t>(m)] = static_cast<int>(g);
    }

    Graph result(graph.name());
    std::vector<NodeId> new_id(graph.num_nodes(), kNoNode);
    std::size_t fused_ops = 0;
    for (std::size_t i = 0; i < graph.num_nodes(); ++i) {
        const Node& node = graph.node(static_cast<NodeId>(i));
        if (group_of[i] < 0) {
            std::vector<NodeId> operands;
            for (NodeId in : node.inputs) operands.push_back(new_id[static_cast<std::size_t>(in)]);
            Result<NodeId> id = result.copy_node(node, std::move(operands));
            if (!id.ok()) return id.error();
            new_id[i] = id.value();
            continue;
        }
        const auto& members = groups[static_cast<std::size_t>(group_of[i])];
        if (static_cast<NodeId>(i) != members.back()) continue;  // the root emits the whole group
        ProgramEmitter emit(graph, new_id);
        for (NodeId m : members) emit.member(m);
        Result<NodeId> id = result.add_fused(emit.externals(), emit.program(), node.type, node.name);
        if (!id.ok()) return id.error();
        new_id[i] = id.value();
        fused_ops += members.size();
    }
    for (NodeId out : graph.outputs()) {
        Status st = result.add_output(new_id[static_cast<std::size_t>(out)]);
        if (!st.ok()) return st.error();
    }
    fill_report(report, "fuse", graph, result,
                "fused " + std::to_string(fused_ops) + " op(s) into " + std::to_string(groups.size()) + " kernel(s)");
    return result;
}

}  // namespace minicompiler
