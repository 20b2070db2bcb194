// FusedProgram checks and printing (the contract of the reference's
// src/fused_program.cpp: instructions read earlier registers only, loads name
// one of the node's inputs, and each op matches its instruction kind; one
// printed line per instruction, "r<i> = <right-hand side>").

#include "minicompiler/fused_program.hpp"

#include <sstream>

namespace minicompiler {

namespace {

// Registers an instruction of kind `k` reads (a, then b).
int registers_read(FusedInstr::Kind k) {
    switch (k) {
        case FusedInstr::Kind::Unary: return 1;
        case FusedInstr::Kind::Binary: return 2;
        default: return 0;
    }
}

// What is wrong with instruction `r`, or "".
std::string instr_problem(const FusedInstr& ins, std::size_t r, std::size_t num_inputs) {
    switch (ins.kind) {
        case FusedInstr::Kind::Load:
            if (ins.a < 0 || static_cast<std::size_t>(ins.a) >= num_inputs) {
                return "load of input " + std::to_string(ins.a) + ", but the node has " + std::to_string(num_inputs);
            }
            return {};
        case FusedInstr::Kind::Immediate: return {};
        case FusedInstr::Kind::Unary:
            if (!is_unary_elementwise(ins.op)) return std::string(op_name(ins.op)) + " is not a unary elementwise op";
            break;
        case FusedInstr::Kind::Binary:
            if (!is_binary_elementwise(ins.op)) return std::string(op_name(ins.op)) + " is not a binary elementwise op";
            break;
        default: return "instruction of unknown kind";
    }
    const std::int32_t regs[2] = {ins.a, ins.b};
    for (int j = 0; j < registers_read(ins.kind); ++j) {
        if (regs[j] < 0 || static_cast<std::size_t>(regs[j]) >= r) {
            return "reads r" + std::to_string(regs[j]) + ", which is not an earlier register";
        }
    }
    return {};
}

void print_rhs(std::ostream& os, const FusedInstr& ins) {
    switch (ins.kind) {
        case FusedInstr::Kind::Load: os << "load in" << ins.a; return;
        case FusedInstr::Kind::Immediate: os << "imm " << ins.immediate; return;
        default: break;
    }
    os << op_name(ins.op) << " r" << ins.a;
    if (registers_read(ins.kind) == 2) os << ", r" << ins.b;
}

}  // namespace

std::size_t FusedProgram::num_ops() const {
    std::size_t ops = 0;
    for (const FusedInstr& ins : instrs) ops += registers_read(ins.kind) > 0 ? 1 : 0;
    return ops;
}

Status validate(const FusedProgram& program, std::size_t num_inputs) {
    if (program.instrs.empty()) return Error{"a fused program needs at least one instruction"};
    for (std::size_t r = 0; r < program.instrs.size(); ++r) {
        const std::string problem = instr_problem(program.instrs[r], r, num_inputs);
        if (!problem.empty()) return Error{"fused instruction r" + std::to_string(r) + ": " + problem};
    }
    return Status();
}

std::string to_string(const FusedProgram& program) {
    std::ostringstream os;
    for (std::size_t r = 0; r < program.instrs.size(); ++r) {
        os << 'r' << r << " = ";
        print_rhs(os, program.instrs[r]);
        os << '\n';
    }
    return os.str();
}

}  // namespace minicompiler
