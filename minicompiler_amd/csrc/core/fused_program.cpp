// FusedProgram checks and printing (reference: src/fused_program.cpp:7-62).

#include "minicompiler/fused_program.hpp"

#include <sstream>

namespace minicompiler {

std::size_t FusedProgram::num_ops() const {
    std::size_t n = 0;
    for (const FusedInstr& ins : instrs) {
        n += ins.kind == FusedInstr::Kind::Unary || ins.kind == FusedInstr::Kind::Binary;
    }
    return n;
}

Status validate(const FusedProgram& program, std::size_t num_inputs) {
    if (program.instrs.empty()) return Error{"fused program is empty"};
    for (std::size_t r = 0; r < program.instrs.size(); ++r) {
        const FusedInstr& ins = program.instrs[r];
        const std::string at = "fused instruction r" + std::to_string(r) + ": ";
        const auto earlier = [r](std::int32_t x) { return x >= 0 && static_cast<std::size_t>(x) < r; };
        switch (ins.kind) {
            case FusedInstr::Kind::Load:
                if (ins.a < 0 || static_cast<std::size_t>(ins.a) >= num_inputs) {
                    return Error{at + "loads input " + std::to_string(ins.a) + " of " + std::to_string(num_inputs)};
                }
                break;
            case FusedInstr::Kind::Immediate:
                break;
            case FusedInstr::Kind::Unary:
                if (!is_unary_elementwise(ins.op)) return Error{at + op_name(ins.op) + " is not a unary elementwise op"};
                if (!earlier(ins.a)) return Error{at + "operand must be an earlier instruction"};
                break;
            case FusedInstr::Kind::Binary:
                if (!is_binary_elementwise(ins.op)) {
                    return Error{at + op_name(ins.op) + " is not a binary elementwise op"};
                }
                if (!earlier(ins.a) || !earlier(ins.b)) return Error{at + "operands must be earlier instructions"};
                break;
            default:
                return Error{at + "unknown instruction kind"};
        }
    }
    return Status();
}

std::string to_string(const FusedProgram& program) {
    std::ostringstream os;
    for (std::size_t r = 0; r < program.instrs.size(); ++r) {
        const FusedInstr& ins = program.instrs[r];
        os << 'r' << r << " = ";
        switch (ins.kind) {
            case FusedInstr::Kind::Load: os << "load in" << ins.a; break;
            case FusedInstr::Kind::Immediate: os << "imm " << ins.immediate; break;
            case FusedInstr::Kind::Unary: os << op_name(ins.op) << " r" << ins.a; break;
            case FusedInstr::Kind::Binary: os << op_name(ins.op) << " r" << ins.a << ", r" << ins.b; break;
        }
        os << '\n';
    }
    return os.str();
}

}  // namespace minicompiler
