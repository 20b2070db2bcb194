#pragma once

// Op kinds and NumPy broadcasting. Same surface as the reference's
// include/minicompiler/ops.hpp:13-72. The numeric values of OpKind are also
// the op codes of the C ABI (include/minicompiler_hip.h) and of the oracle.

#include "minicompiler/result.hpp"
#include "minicompiler/tensor.hpp"

#include <cstdint>
#include <optional>
#include <string_view>
#include <vector>

namespace minicompiler {

enum class OpKind : std::uint8_t {
    Input = 0,     // runtime argument
    Constant = 1,  // value known at compile time
    // unary elementwise
    Neg = 2,
    Exp = 3,
    Log = 4,
    Sqrt = 5,
    Relu = 6,
    Sigmoid = 7,
    Tanh = 8,
    // binary elementwise, NumPy broadcasting
    Add = 9,
    Sub = 10,
    Mul = 11,
    Div = 12,
    // [M,K] x [K,N] -> [M,N]
    MatMul = 13,
    // several elementwise ops run as one generated kernel (see FusedProgram)
    FusedElementwise = 14,
};

const char* op_name(OpKind op);

// Only the ops a graph file can spell as `name = op a, b` are found.
std::optional<OpKind> op_from_name(std::string_view name);

bool is_unary_elementwise(OpKind op);
bool is_binary_elementwise(OpKind op);
inline bool is_elementwise(OpKind op) { return is_unary_elementwise(op) || is_binary_elementwise(op); }
inline bool is_compute(OpKind op) { return op != OpKind::Input && op != OpKind::Constant; }

// Operand count; -1 for FusedElementwise (variable).
int op_arity(OpKind op);

Result<Shape> broadcast_shapes(const Shape& a, const Shape& b);

// Per output dimension, the element stride of `in` when read at the output's
// coordinates: 0 along broadcast dimensions.
std::vector<std::int64_t> broadcast_strides(const Shape& in, const Shape& out);

Result<TensorType> infer_result_type(OpKind op, const std::vector<TensorType>& operands);

}  // namespace minicompiler
