#pragma once

// The per-element program of a FusedElementwise node. Same contract as the
// reference's include/minicompiler/fused_program.hpp:16-52: a tiny SSA
// program evaluated once per output element, one float register per
// instruction, operands naming earlier instructions; the last one is the
// result.

#include "minicompiler/ops.hpp"
#include "minicompiler/result.hpp"

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace minicompiler {

struct FusedInstr {
    enum class Kind : std::uint8_t {
        Load = 0,       // element of fused input `a`, broadcast to the output shape
        Immediate = 1,  // the constant `immediate`
        Unary = 2,      // op(r[a])
        Binary = 3,     // op(r[a], r[b])
    };

    Kind kind = Kind::Load;
    OpKind op = OpKind::Input;
    std::int32_t a = -1;
    std::int32_t b = -1;
    float immediate = 0.0f;

    static FusedInstr load(std::int32_t input) { return {Kind::Load, OpKind::Input, input, -1, 0.0f}; }
    static FusedInstr imm(float value) { return {Kind::Immediate, OpKind::Constant, -1, -1, value}; }
    static FusedInstr unary(OpKind op, std::int32_t x) { return {Kind::Unary, op, x, -1, 0.0f}; }
    static FusedInstr binary(OpKind op, std::int32_t x, std::int32_t y) { return {Kind::Binary, op, x, y, 0.0f}; }
};

struct FusedProgram {
    std::vector<FusedInstr> instrs;
    // Names of the graph nodes the program replaces, in program order.
    std::vector<std::string> source_nodes;

    // Unary + Binary instructions.
    std::size_t num_ops() const;
};

// Operands name earlier registers, loads name one of `num_inputs` inputs,
// ops have the right arity.
Status validate(const FusedProgram& program, std::size_t num_inputs);

// One instruction per line: "r2 = mul r0, r1".
std::string to_string(const FusedProgram& program);

}  // namespace minicompiler
