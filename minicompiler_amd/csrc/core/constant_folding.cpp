// Constant folding (reference: src/passes/constant_folding.cpp:10-51) and the
// host evaluator it uses. The reference folds with its Eigen CPU kernels;
// this library evaluates on the host with the same per-operation float
// semantics: every op's result is rounded to float, binary ops broadcast
// NumPy-style, a matmul accumulates in float along K, and a fused program is
// evaluated per element with float registers. Only compile-time constants
// (at most max_elements per node) are evaluated here; nothing at run time.

#include "minicompiler/passes/constant_folding.hpp"

#include <algorithm>
#include <cmath>
#include <vector>

namespace minicompiler {

namespace {

float unary_value(OpKind op, float x) {
    switch (op) {
        case OpKind::Neg: return -x;
        case OpKind::Exp: return std::exp(x);
        case OpKind::Log: return std::log(x);
        case OpKind::Sqrt: return std::sqrt(x);
        case OpKind::Relu: return x > 0.0f ? x : 0.0f;
        case OpKind::Sigmoid: {
            const float d = 1.0f + std::exp(-x);
            return 1.0f / d;
        }
        case OpKind::Tanh: return std::tanh(x);
        default: return std::nanf("");
    }
}

float binary_value(OpKind op, float a, float b) {
    switch (op) {
        case OpKind::Add: return a + b;
        case OpKind::Sub: return a - b;
        case OpKind::Mul: return a * b;
        case OpKind::Div: return a / b;
        default: return std::nanf("");
    }
}

// Element offset into an operand read with `strides` at output position i.
std::int64_t operand_offset(std::size_t i, const Shape& out, const std::vector<std::int64_t>& strides) {
    std::int64_t off = 0;
    for (std::size_t d = out.size(); d-- > 0;) {
        const auto extent = static_cast<std::size_t>(out[d]);
        off += static_cast<std::int64_t>(i % extent) * strides[d];
        i /= extent;
    }
    return off;
}

}  // namespace

void fold_evaluate_node(const Node& node, const std::vector<const float*>& operands,
                        const std::vector<Shape>& operand_shapes, float* out) {
    const Shape& shape = node.type.shape;
    const std::size_t n = node.type.num_elements();
    if (is_unary_elementwise(node.op)) {
        for (std::size_t i = 0; i < n; ++i) out[i] = unary_value(node.op, operands[0][i]);
    } else if (is_binary_elementwise(node.op)) {
        const auto sa = broadcast_strides(operand_shapes[0], shape);
        const auto sb = broadcast_strides(operand_shapes[1], shape);
        for (std::size_t i = 0; i < n; ++i) {
            out[i] = binary_value(node.op, operands[0][operand_offset(i, shape, sa)],
                                  operands[1][operand_offset(i, shape, sb)]);
        }
    } else if (node.op == OpKind::MatMul) {
        const std::int64_t m = operand_shapes[0][0], k = operand_shapes[0][1], cols = operand_shapes[1][1];
        std::fill(out, out + n, 0.0f);
        for (std::int64_t r = 0; r < m; ++r) {
            float* row = out + r * cols;
            for (std::int64_t t = 0; t < k; ++t) {
                const float a = operands[0][r * k + t];
                const float* b = operands[1] + t * cols;
                for (std::int64_t c = 0; c < cols; ++c) {
                    const float p = a * b[c];
                    row[c] = row[c] + p;
                }
            }
        }
    } else if (node.op == OpKind::FusedElementwise) {
        const FusedProgram& p = *node.fused;
        std::vector<std::vector<std::int64_t>> strides;
        for (const Shape& s : operand_shapes) strides.push_back(broadcast_strides(s, shape));
        std::vector<float> r(p.instrs.size());
        for (std::size_t i = 0; i < n; ++i) {
            for (std::size_t j = 0; j < p.instrs.size(); ++j) {
                const FusedInstr& ins = p.instrs[j];
                switch (ins.kind) {
                    case FusedInstr::Kind::Load: {
                        const auto in = static_cast<std::size_t>(ins.a);
                        r[j] = operands[in][operand_offset(i, shape, strides[in])];
                        break;
                    }
                    case FusedInstr::Kind::Immediate: r[j] = ins.immediate; break;
                    case FusedInstr::Kind::Unary: r[j] = unary_value(ins.op, r[ins.a]); break;
                    case FusedInstr::Kind::Binary: r[j] = binary_value(ins.op, r[ins.a], r[ins.b]); break;
                }
            }
            out[i] = r.back();
        }
    }
}

Result<Graph> fold_constants(const Graph& graph, PassReport* report, const ConstantFoldingOptions& options) {
    Graph result(graph.name());
    std::vector<NodeId> new_id(graph.num_nodes(), kNoNode);
    std::size_t folded = 0;
    for (std::size_t i = 0; i < graph.num_nodes(); ++i) {
        const Node& node = graph.node(static_cast<NodeId>(i));
        std::vector<NodeId> operands;
        for (NodeId in : node.inputs) operands.push_back(new_id[static_cast<std::size_t>(in)]);
        bool foldable = is_compute(node.op) && !operands.empty() && node.type.num_elements() <= options.max_elements;
        for (NodeId in : operands) foldable = foldable && result.node(in).op == OpKind::Constant;
        if (foldable) {
            std::vector<const float*> values;
            std::vector<Shape> shapes;
            for (NodeId in : operands) {
                values.push_back(result.node(in).constant->data());
                shapes.push_back(result.node(in).type.shape);
            }
            std::vector<float> out(node.type.num_elements());
            fold_evaluate_node(node, values, shapes, out.data());
            Result<NodeId> id = result.add_constant(node.name, node.type, std::move(out));
            if (!id.ok()) return id.error();
            new_id[i] = id.value();
            ++folded;
            continue;
        }
        Result<NodeId> id = result.copy_node(node, std::move(operands));
        if (!id.ok()) return id.error();
        new_id[i] = id.value();
    }
    for (NodeId out : graph.outputs()) {
        Status st = result.add_output(new_id[static_cast<std::size_t>(out)]);
        if (!st.ok()) return st.error();
    }
    fill_report(report, "fold", graph, result, "folded " + std::to_string(folded) + " node(s) into constants");
    return result;
}

}  // namespace minicompiler
