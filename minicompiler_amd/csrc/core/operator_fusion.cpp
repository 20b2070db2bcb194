// Elementwise fusion (the contract of the reference's
// src/passes/operator_fusion.cpp: which nodes share a kernel and the order of
// the instructions in each program are pinned by the reference's known
// answers, e.g. the GELU chain's one load and four immediates).
//
// Groups. Roots are taken from the highest unassigned elementwise id down.
// From a root the group grows toward its producers: the ids below it are
// swept downward, and an id the group reads (a candidate) joins when it is
// an unassigned elementwise node of the root's shape, not a graph output,
// whose every reader is already in the group. Its operands become
// candidates. A node's readers all have higher ids, so the downward sweep
// decides every reader before the node itself: the group is closed under
// "all readers inside", and no value it computes leaves the kernel.
//
// Programs. Members are emitted in ascending id order. A member's operands
// get registers the first time they are read, operand a before operand b: a
// member computed earlier in the group is its register, a one-element
// constant becomes an immediate, anything else a load of the next external
// input.

#include "minicompiler/passes/operator_fusion.hpp"

#include <algorithm>
#include <memory>

namespace minicompiler {

std::vector<std::vector<NodeId>> find_fusion_groups(const Graph& graph) {
    const std::size_t n = graph.num_nodes();
    const std::vector<std::vector<NodeId>> readers = graph.compute_users();
    std::vector<int> group_of(n, -1);
    std::vector<char> wanted(n, 0);  // read by the group being grown
    std::vector<std::vector<NodeId>> by_root;  // highest root first

    for (std::size_t r = n; r-- > 0;) {
        const Node& root = graph.node(static_cast<NodeId>(r));
        if (!is_elementwise(root.op) || group_of[r] >= 0) continue;
        const int g = static_cast<int>(by_root.size());
        group_of[r] = g;
        std::vector<NodeId> members{static_cast<NodeId>(r)};
        std::size_t lowest = r;  // no candidate lies below it
        auto want_operands = [&](const Node& m) {
            for (NodeId in : m.inputs) {
                wanted[static_cast<std::size_t>(in)] = 1;
                lowest = std::min(lowest, static_cast<std::size_t>(in));
            }
        };
        want_operands(root);
        for (std::size_t p = r; p-- > lowest;) {
            if (!wanted[p]) continue;
            wanted[p] = 0;
            const Node& pn = graph.node(static_cast<NodeId>(p));
            if (group_of[p] >= 0 || !is_elementwise(pn.op) || pn.type.shape != root.type.shape ||
                graph.is_output(static_cast<NodeId>(p))) {
                continue;
            }
            bool enclosed = true;
            for (NodeId u : readers[p]) enclosed = enclosed && group_of[static_cast<std::size_t>(u)] == g;
            if (!enclosed) continue;
            group_of[p] = g;
            members.push_back(static_cast<NodeId>(p));
            want_operands(pn);
        }
        // Every mark lay in [lowest, r) and the sweep cleared it on its way down.
        std::vector<NodeId> ascending(members.rbegin(), members.rend());
        by_root.push_back(std::move(ascending));
    }

    std::vector<std::vector<NodeId>> groups;  // lowest root first, singletons dropped
    for (std::size_t i = by_root.size(); i-- > 0;) {
        if (by_root[i].size() >= 2) groups.push_back(std::move(by_root[i]));
    }
    return groups;
}

namespace {

struct EmittedGroup {
    std::shared_ptr<FusedProgram> program = std::make_shared<FusedProgram>();
    std::vector<NodeId> externals;  // operand ids in the new graph, in load order
};

// The FusedProgram of one group (members ascending). `new_id` maps old ids
// of already rebuilt nodes to the new graph's.
EmittedGroup emit_group(const Graph& graph, const std::vector<NodeId>& members, const std::vector<NodeId>& new_id) {
    EmittedGroup out;
    std::vector<std::pair<NodeId, std::int32_t>> regs;  // node -> register, in emission order
    auto append = [&](NodeId id, const FusedInstr& ins) {
        out.program->instrs.push_back(ins);
        const auto r = static_cast<std::int32_t>(out.program->instrs.size() - 1);
        regs.emplace_back(id, r);
        return r;
    };
    auto operand = [&](NodeId id) -> std::int32_t {
        for (const auto& [node, r] : regs) {
            if (node == id) return r;
        }
        const Node& src = graph.node(id);
        if (src.op == OpKind::Constant && src.type.num_elements() == 1) {
            return append(id, FusedInstr::imm((*src.constant)[0]));
        }
        out.externals.push_back(new_id[static_cast<std::size_t>(id)]);
        return append(id, FusedInstr::load(static_cast<std::int32_t>(out.externals.size() - 1)));
    };
    for (NodeId m : members) {
        const Node& node = graph.node(m);
        const std::int32_t a = operand(node.inputs[0]);
        if (is_binary_elementwise(node.op)) {
            const std::int32_t b = operand(node.inputs[1]);
            append(m, FusedInstr::binary(node.op, a, b));
        } else {
            append(m, FusedInstr::unary(node.op, a));
        }
        out.program->source_nodes.push_back(node.name);
    }
    return out;
}

}  // namespace

Result<Graph> fuse_elementwise(const Graph& graph, PassReport* report) {
    const std::vector<std::vector<NodeId>> groups = find_fusion_groups(graph);
    // root_of[v]: the group whose last (root) member is v; member[v]: v is in a group.
    std::vector<int> root_of(graph.num_nodes(), -1);
    std::vector<char> member(graph.num_nodes(), 0);
    std::size_t fused_ops = 0;
    for (std::size_t g = 0; g < groups.size(); ++g) {
        for (NodeId m : groups[g]) member[static_cast<std::size_t>(m)] = 1;
        root_of[static_cast<std::size_t>(groups[g].back())] = static_cast<int>(g);
        fused_ops += groups[g].size();
    }

    Graph result(graph.name());
    std::vector<NodeId> new_id(graph.num_nodes(), kNoNode);
    for (std::size_t i = 0; i < graph.num_nodes(); ++i) {
        const Node& node = graph.node(static_cast<NodeId>(i));
        Result<NodeId> id = kNoNode;
        if (root_of[i] >= 0) {
            EmittedGroup e = emit_group(graph, groups[static_cast<std::size_t>(root_of[i])], new_id);
            id = result.add_fused(std::move(e.externals), std::move(e.program), node.type, node.name);
        } else if (!member[i]) {
            std::vector<NodeId> operands;
            for (NodeId in : node.inputs) operands.push_back(new_id[static_cast<std::size_t>(in)]);
            id = result.copy_node(node, std::move(operands));
        } else {
            continue;  // computed inside its group's kernel
        }
        if (!id.ok()) return id.error();
        new_id[i] = id.value();
    }
    for (NodeId out : graph.outputs()) {
        if (Status st = result.add_output(new_id[static_cast<std::size_t>(out)]); !st.ok()) return st.error();
    }
    fill_report(report, "fuse", graph, result,
                "fused " + std::to_string(fused_ops) + " op(s) into " + std::to_string(groups.size()) + " kernel(s)");
    return result;
}

}  // namespace minicompiler
