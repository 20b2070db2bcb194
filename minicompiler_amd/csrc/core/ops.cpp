// Op names, arities and NumPy broadcasting (reference: src/ops.cpp:8-134).

#include "minicompiler/ops.hpp"

#include <algorithm>
#include <string>

namespace minicompiler {

namespace {

struct OpInfo {
    OpKind op;
    const char* name;
    int arity;  // -1: variable
    bool writable;  // spelled `y = name a[, b]` in a graph file
};

constexpr OpInfo kOps[] = {
    {OpKind::Input, "input", 0, false},     {OpKind::Constant, "const", 0, false},
    {OpKind::Neg, "neg", 1, true},          {OpKind::Exp, "exp", 1, true},
    {OpKind::Log, "log", 1, true},          {OpKind::Sqrt, "sqrt", 1, true},
    {OpKind::Relu, "relu", 1, true},        {OpKind::Sigmoid, "sigmoid", 1, true},
    {OpKind::Tanh, "tanh", 1, true},        {OpKind::Add, "add", 2, true},
    {OpKind::Sub, "sub", 2, true},          {OpKind::Mul, "mul", 2, true},
    {OpKind::Div, "div", 2, true},          {OpKind::MatMul, "matmul", 2, true},
    {OpKind::FusedElementwise, "fused", -1, false},
};

const OpInfo* info(OpKind op) {
    const auto i = static_cast<std::size_t>(op);
    return i < sizeof(kOps) / sizeof(kOps[0]) ? &kOps[i] : nullptr;
}

}  // namespace

const char* op_name(OpKind op) {
    const OpInfo* i = info(op);
    return i ? i->name : "?";
}

std::optional<OpKind> op_from_name(std::string_view name) {
    for (const OpInfo& i : kOps) {
        if (i.writable && name == i.name) return i.op;
    }
    return std::nullopt;
}

bool is_unary_elementwise(OpKind op) { return op >= OpKind::Neg && op <= OpKind::Tanh; }

bool is_binary_elementwise(OpKind op) { return op >= OpKind::Add && op <= OpKind::Div; }

int op_arity(OpKind op) {
    const OpInfo* i = info(op);
    return i ? i->arity : -1;
}

Result<Shape> broadcast_shapes(const Shape& a, const Shape& b) {
    const std::size_t rank = std::max(a.size(), b.size());
    Shape out(rank, 1);
    // Align on the right; a missing leading dimension acts as 1.
    for (std::size_t r = 0; r < rank; ++r) {
        const std::int64_t da = r < a.size() ? a[a.size() - 1 - r] : 1;
        const std::int64_t db = r < b.size() ? b[b.size() - 1 - r] : 1;
        if (da != db && da != 1 && db != 1) {
            return Error{"cannot broadcast " + to_string(a) + " with " + to_string(b)};
        }
        out[rank - 1 - r] = da == 1 ? db : da;
    }
    return out;
}

std::vector<std::int64_t> broadcast_strides(const Shape& in, const Shape& out) {
    std::vector<std::int64_t> strides(out.size(), 0);
    std::int64_t step = 1;
    for (std::size_t r = 0; r < in.size(); ++r) {
        const std::int64_t dim = in[in.size() - 1 - r];
        if (dim != 1) strides[out.size() - 1 - r] = step;
        step *= dim;
    }
    return strides;
}

Result<TensorType> infer_result_type(OpKind op, const std::vector<TensorType>& operands) {
    const int arity = op_arity(op);
    if (arity <= 0) return Error{std::string("'") + op_name(op) + "' has no inferred result type"};
    if (operands.size() != static_cast<std::size_t>(arity)) {
        return Error{std::string(op_name(op)) + " expects " + std::to_string(arity) + " operand(s), got " +
                     std::to_string(operands.size())};
    }
    for (const TensorType& t : operands) {
        if (t.dtype != DType::Float32) {
            return Error{std::string(op_name(op)) + ": only f32 is supported, got " + to_string(t)};
        }
    }
    if (is_unary_elementwise(op)) return operands[0];
    if (is_binary_elementwise(op)) {
        Result<Shape> s = broadcast_shapes(operands[0].shape, operands[1].shape);
        if (!s.ok()) return Error{std::string(op_name(op)) + ": " + s.error().message};
        return TensorType(std::move(s).value());
    }
    const Shape& a = operands[0].shape;
    const Shape& b = operands[1].shape;
    if (a.size() != 2 || b.size() != 2) {
        return Error{"matmul expects rank-2 operands, got " + to_string(a) + " and " + to_string(b)};
    }
    if (a[1] != b[0]) return Error{"matmul inner dimensions differ: " + to_string(a) + " x " + to_string(b)};
    return TensorType({a[0], b[1]});
}

}  // namespace minicompiler
