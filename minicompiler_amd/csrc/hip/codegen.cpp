// HIP C++ generator for elementwise kernels on gfx950 (replaces the
// reference's src/cuda/codegen.cpp:14-182; the access classes and the
// vectorisation rule are the reference's, the kernel shape is CDNA4's).
//
// Kernel shape. A block is 256 lanes (four wave64s). Each lane owns
// `items_per_lane` items (16-byte vectors when vectorised) spaced one block
// apart, so every load instruction of a wave reads 1 KiB of consecutive
// memory. A lane issues all its loads, then evaluates the program per float,
// then issues all its stores: U x 16 bytes in flight per lane. The grid
// walks the tensor in block-sized steps of 256 x U items; steps where a lane's
// items are all in range take the unchecked path, the single ragged step the
// checked one.
//
// Numerics. The program is a device function of the inputs' floats: one
// `const float` per instruction, so with -ffp-contract=off every op rounds
// to float, as the reference's per-instruction register semantics require.
// Immediates are written as their exact bit patterns.

#include "codegen.hpp"

#include "rtc_sources.hpp"

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <sstream>
#include <utility>

namespace minicompiler::hip {

namespace {

std::string exact_float(float v) {
    std::uint32_t bits = 0;
    std::memcpy(&bits, &v, sizeof bits);
    char buf[96];
    std::snprintf(buf, sizeof buf, "__uint_as_float(0x%08xu) /* %.9g */", static_cast<unsigned>(bits),
                  static_cast<double>(v));
    return buf;
}

std::string op_text(OpKind op, const std::string& a, const std::string& b) {
    switch (op) {
        case OpKind::Neg: return "-" + a;
        case OpKind::Exp: return "expf(" + a + ")";
        case OpKind::Log: return "logf(" + a + ")";
        case OpKind::Sqrt: return "sqrtf(" + a + ")";
        case OpKind::Relu: return "fmaxf(" + a + ", 0.0f)";
        case OpKind::Sigmoid: return "1.0f / (1.0f + expf(-" + a + "))";
        case OpKind::Tanh: return "mc_tanh(" + a + ")";
        case OpKind::Add: return a + " + " + b;
        case OpKind::Sub: return a + " - " + b;
        case OpKind::Mul: return a + " * " + b;
        case OpKind::Div: return a + " / " + b;
        default: return "__builtin_nanf(\"\") /* not an elementwise op */";
    }
}

std::string u32(std::size_t v) { return std::to_string(v) + "u"; }

// tanh in about 15 VALU instructions instead of the library's ~25, which
// matters for GELU-shaped groups at HBM speed. For |x| < 0.625 an odd
// polynomial x + x^3 P(x^2), P of degree 4 fitted here for relative error on
// [0, 0.625] (7.6e-8 worst over every float of the range, in this float
// arithmetic); above, 1 - 2 / (e^{2|x|} + 1) with the hardware exp2 and
// reciprocal (2.7e-7 worst with both off by one ulp) and the sign of x.
// The sign of x is applied last (so tanh(-0) is -0). NaN, +-0 and +-inf
// behave as tanhf does.
const char* const kTanhSource = R"(__device__ __forceinline__ float mc_tanh(float x)
{
	const float z = x * x;
	float p = __uint_as_float(0xbbbaf0eau) /* -0.00570498873 */;
	p = fmaf(p, z, __uint_as_float(0x3ca9134fu) /* 0.0206390899 */);
	p = fmaf(p, z, __uint_as_float(0xbd5c1e2du) /* -0.0537397154 */);
	p = fmaf(p, z, __uint_as_float(0x3e088393u) /* 0.133314416 */);
	p = fmaf(p, z, __uint_as_float(0xbeaaaa99u) /* -0.333332807 */);
	const float xz = x * z;
	const float small = fmaf(xz, p, x);
	const float a = fabsf(x);
	const float t = __builtin_amdgcn_exp2f(a * __uint_as_float(0x4038aa3bu) /* 2 log2(e) */);
	const float r = __builtin_amdgcn_rcpf(t + 1.0f);
	const float big = fmaf(-2.0f, r, 1.0f);
	return copysignf(a < 0.625f ? small : big, x);
}

)";

// 1 + tanh(x) = 2 / (1 + e^{-2x}): one exp2 and one reciprocal, and no
// cancellation as tanh(x) -> -1 (1 + tanh(x) computed in float loses every
// significant bit there). About 3 ulp from the exact value.
const char* const kOnePlusTanhSource = R"(__device__ __forceinline__ float mc_one_plus_tanh(float x)
{
	const float e = __builtin_amdgcn_exp2f(x * __uint_as_float(0xc038aa3bu) /* -2 log2(e) */);
	return 2.0f * __builtin_amdgcn_rcpf(1.0f + e);
}

)";

// (1 + tanh(x)) / 2 = 1 / (1 + e^{-2x}): the same exp2 and reciprocal as
// mc_one_plus_tanh, without its doubling.
const char* const kHalfOnePlusTanhSource = R"(__device__ __forceinline__ float mc_half_one_plus_tanh(float x)
{
	const float e = __builtin_amdgcn_exp2f(x * __uint_as_float(0xc038aa3bu) /* -2 log2(e) */);
	return __builtin_amdgcn_rcpf(1.0f + e);
}

)";

// How each instruction of a program is emitted.
struct Form {
    enum class Kind : std::uint8_t { Plain, Absorbed, OnePlusTanh, HalfOnePlusTanh, Fma } kind = Kind::Plain;
    // OnePlusTanh: x = tanh's operand. HalfOnePlusTanh: x * mc_half_one_plus_tanh(y).
    // Fma: x * y + z (with `neg_x`: -x * y + z, `neg_z`: x * y - z).
    std::int32_t x = -1, y = -1, z = -1;
    bool neg_x = false, neg_z = false;
};

// Forms of the instructions of a multi-op program (a single op is emitted
// as it is, so it rounds exactly as the reference's op does):
// - an add of the immediate 1.0 and a tanh used only there becomes
//   mc_one_plus_tanh of the tanh's operand;
// - a mul of such a sum (used only there) by x * 0.5 (used only there), the
//   tail of GELU, becomes x * mc_half_one_plus_tanh: (x / 2)(2 r) is x r
//   exactly wherever x / 2 is exact (all but |x| < 2^-125), two multiplies
//   fewer per element;
// - a mul used only by one add or sub becomes an fmaf there (one rounding
//   instead of two), as NVRTC contracts a*b+c by default: the reference's
//   run-time compile passes no option against it (src/cuda/kernel_compiler.cpp:35-37).
std::vector<Form> program_forms(const FusedProgram& program) {
    const std::size_t n = program.instrs.size();
    std::vector<Form> forms(n);
    if (program.num_ops() < 2) return forms;
    std::vector<int> uses(n, 0);
    for (const FusedInstr& ins : program.instrs) {
        if (ins.kind == FusedInstr::Kind::Unary || ins.kind == FusedInstr::Kind::Binary) ++uses[ins.a];
        if (ins.kind == FusedInstr::Kind::Binary) ++uses[ins.b];
    }
    ++uses[n - 1];
    auto is = [&](std::int32_t r, OpKind op, FusedInstr::Kind kind) {
        const FusedInstr& i = program.instrs[r];
        return i.kind == kind && i.op == op && uses[r] == 1 && forms[r].kind == Form::Kind::Plain;
    };
    auto is_one = [&](std::int32_t r) {
        const FusedInstr& i = program.instrs[r];
        return i.kind == FusedInstr::Kind::Immediate && i.immediate == 1.0f;
    };
    for (std::size_t r = 0; r < n; ++r) {
        const FusedInstr& ins = program.instrs[r];
        if (ins.kind != FusedInstr::Kind::Binary) continue;
        Form& f = forms[r];
        if (ins.op == OpKind::Add) {
            for (const auto& [t, k] : {std::pair{ins.a, ins.b}, std::pair{ins.b, ins.a}}) {
                if (is(t, OpKind::Tanh, FusedInstr::Kind::Unary) && is_one(k)) {
                    f = {Form::Kind::OnePlusTanh, program.instrs[t].a};
                    forms[t].kind = Form::Kind::Absorbed;
                    break;
                }
            }
            if (f.kind != Form::Kind::Plain) continue;
            for (const auto& [m, z] : {std::pair{ins.a, ins.b}, std::pair{ins.b, ins.a}}) {
                if (is(m, OpKind::Mul, FusedInstr::Kind::Binary)) {
                    f = {Form::Kind::Fma, program.instrs[m].a, program.instrs[m].b, z};
                    forms[m].kind = Form::Kind::Absorbed;
                    break;
                }
            }
        } else if (ins.op == OpKind::Sub) {
            if (is(ins.a, OpKind::Mul, FusedInstr::Kind::Binary)) {  // x y - z
                f = {Form::Kind::Fma, program.instrs[ins.a].a, program.instrs[ins.a].b, ins.b, false, true};
                forms[ins.a].kind = Form::Kind::Absorbed;
            } else if (is(ins.b, OpKind::Mul, FusedInstr::Kind::Binary)) {  // z - x y
                f = {Form::Kind::Fma, program.instrs[ins.b].a, program.instrs[ins.b].b, ins.a, true, false};
                forms[ins.b].kind = Form::Kind::Absorbed;
            }
        }
    }
    // (x * 0.5) * (1 + tanh u), each factor used only there.
    auto is_half = [&](std::int32_t r) {
        const FusedInstr& i = program.instrs[r];
        return i.kind == FusedInstr::Kind::Immediate && i.immediate == 0.5f;
    };
    for (std::size_t r = 0; r < n; ++r) {
        const FusedInstr& ins = program.instrs[r];
        if (ins.kind != FusedInstr::Kind::Binary || ins.op != OpKind::Mul || forms[r].kind != Form::Kind::Plain) continue;
        for (const auto& [p, h] : {std::pair{ins.a, ins.b}, std::pair{ins.b, ins.a}}) {
            if (p == h || forms[p].kind != Form::Kind::OnePlusTanh || uses[p] != 1) continue;
            if (!is(h, OpKind::Mul, FusedInstr::Kind::Binary)) continue;
            const FusedInstr& hm = program.instrs[h];
            const std::int32_t x = is_half(hm.b) ? hm.a : is_half(hm.a) ? hm.b : -1;
            if (x < 0) continue;
            forms[r] = {Form::Kind::HalfOnePlusTanh, x, forms[p].x};
            forms[p].kind = Form::Kind::Absorbed;
            forms[h].kind = Form::Kind::Absorbed;
            break;
        }
    }
    return forms;
}

// The program as a device function of its inputs' floats, preceded by the
// helper functions it calls: one `const float` per instruction, so with
// -ffp-contract=off every op rounds to float, except where program_forms
// fuses two instructions into one.
std::string program_function(const FusedProgram& program, std::size_t num_inputs) {
    const std::vector<Form> forms = program_forms(program);
    bool tanh = false, one_plus_tanh = false, half_one_plus_tanh = false;
    std::ostringstream body;
    auto reg = [](std::int32_t r) { return "r" + std::to_string(r); };
    for (std::size_t r = 0; r < program.instrs.size(); ++r) {
        const FusedInstr& ins = program.instrs[r];
        const Form& f = forms[r];
        if (f.kind == Form::Kind::Absorbed) continue;
        body << "\tconst float r" << r << " = ";
        if (f.kind == Form::Kind::OnePlusTanh) {
            one_plus_tanh = true;
            body << "mc_one_plus_tanh(" << reg(f.x) << ")";
        } else if (f.kind == Form::Kind::HalfOnePlusTanh) {
            half_one_plus_tanh = true;
            body << reg(f.x) << " * mc_half_one_plus_tanh(" << reg(f.y) << ")";
        } else if (f.kind == Form::Kind::Fma) {
            body << "fmaf(" << (f.neg_x ? "-" : "") << reg(f.x) << ", " << reg(f.y) << ", " << (f.neg_z ? "-" : "")
                 << reg(f.z) << ")";
        } else {
            switch (ins.kind) {
                case FusedInstr::Kind::Load: body << "x" << ins.a; break;
                case FusedInstr::Kind::Immediate: body << exact_float(ins.immediate); break;
                case FusedInstr::Kind::Unary:
                    tanh = tanh || ins.op == OpKind::Tanh;
                    body << op_text(ins.op, reg(ins.a), "");
                    break;
                case FusedInstr::Kind::Binary: body << op_text(ins.op, reg(ins.a), reg(ins.b)); break;
            }
        }
        body << ";\n";
    }
    std::ostringstream os;
    if (tanh) os << kTanhSource;
    if (one_plus_tanh) os << kOnePlusTanhSource;
    if (half_one_plus_tanh) os << kHalfOnePlusTanhSource;
    os << "__device__ __forceinline__ float mc_program(";
    for (std::size_t k = 0; k < num_inputs; ++k) os << (k ? ", " : "") << "float x" << k;
    if (num_inputs == 0) os << "void";
    os << ")\n{\n" << body.str();
    os << "\treturn r" << program.instrs.size() - 1 << ";\n}\n\n";
    return os.str();
}

}  // namespace

Access classify_access(const Shape& in, const Shape& out) {
    const std::size_t count = num_elements(in);
    if (count == 1) return {Access::Kind::Scalar, 0, ""};
    if (count == num_elements(out)) return {Access::Kind::Contiguous, 0, ""};
    // Leading 1s dropped, the rest equal to the output's trailing dims: the
    // input repeats every `count` output elements.
    std::size_t lead = 0;
    while (lead < in.size() && in[lead] == 1) ++lead;
    const std::size_t rest = in.size() - lead;
    if (rest <= out.size() && std::equal(in.begin() + static_cast<std::ptrdiff_t>(lead), in.end(),
                                         out.end() - static_cast<std::ptrdiff_t>(rest))) {
        return {Access::Kind::Periodic, count, ""};
    }
    // sum over broadcast-free dims d of coord_d * stride_d, with
    // coord_d = (i / out_stride_d) % out_d (the outermost never wraps).
    const std::vector<std::int64_t> strides = broadcast_strides(in, out);
    std::vector<std::size_t> out_stride(out.size());
    std::size_t s = 1;
    for (std::size_t d = out.size(); d-- > 0;) {
        out_stride[d] = s;
        s *= static_cast<std::size_t>(out[d]);
    }
    std::string expr;
    for (std::size_t d = 0; d < out.size(); ++d) {
        if (strides[d] == 0) continue;
        std::string coord = out_stride[d] == 1 ? "i" : "(i / " + u32(out_stride[d]) + ")";
        if (d > 0) coord = "(" + coord + " % " + u32(static_cast<std::size_t>(out[d])) + ")";
        if (strides[d] != 1) coord += " * " + u32(static_cast<std::size_t>(strides[d]));
        expr += (expr.empty() ? "" : " + ") + coord;
    }
    return {Access::Kind::General, 0, expr};
}

GemmEpilogueKernel generate_gemm_epilogue_kernel(const FusedProgram& program, std::size_t acc_input,
                                                 const std::vector<Shape>& input_shapes, const Shape& out_shape,
                                                 bool vectorized_operands, const char* gemm_body_source,
                                                 GemmBody body, const GemmDims& fixed) {
    const std::size_t num_inputs = input_shapes.size();
    std::ostringstream os;
    os << "// minicompiler-hip " << (is_f32_body(body) ? "FP32" : body == GemmBody::Bf16Fast ? "bf16" : "fp16")
       << " GEMM with a fused epilogue: " << program.num_ops() << " op(s) on the result, out f32"
       << to_string(out_shape) << ".\n";
    // The ring and narrow bodies add split-K partials in the launch through
    // mc_split_last_arrival.
    const bool folds = is_f32_body(body) && body != GemmBody::F32Mfma;
    if (folds) os << kGemmSplitArrivalSource << "\n";
    os << gemm_body_source << "\n";
    os << program_function(program, num_inputs);
    // Index helpers of General inputs, in terms of the flat output index i.
    for (std::size_t k = 0; k < num_inputs; ++k) {
        if (k == acc_input) continue;
        const Access a = classify_access(input_shapes[k], out_shape);
        if (a.kind == Access::Kind::General) {
            os << "__device__ __forceinline__ unsigned mc_general_" << k << "(unsigned i) { return " << a.index
               << "; }\n";
        }
    }
    // The epilogue: input `acc_input` is the GEMM's value, the others are read
    // at flat output index i by their access class.
    os << "struct McEpilogue\n{\n";
    for (std::size_t k = 0; k < num_inputs; ++k) os << "\tconst float* __restrict__ in" << k << ";\n";
    os << "\t__device__ __forceinline__ float operator()(float v, unsigned i) const\n\t{\n\t\treturn mc_program(";
    for (std::size_t k = 0; k < num_inputs; ++k) {
        if (k) os << ", ";
        if (k == acc_input) {
            os << "v";
            continue;
        }
        const Access a = classify_access(input_shapes[k], out_shape);
        switch (a.kind) {
            case Access::Kind::Scalar: os << "in" << k << "[0]"; break;
            case Access::Kind::Contiguous: os << "in" << k << "[i]"; break;
            case Access::Kind::Periodic: os << "in" << k << "[i % " << u32(a.period) << "]"; break;
            case Access::Kind::General: os << "in" << k << "[mc_general_" << k << "(i)]"; break;
        }
    }
    os << ");\n\t}\n};\n\n";
    // The body's shape arguments: the kernel's own, or constants.
    const bool constant = fixed.m > 0;
    const std::string mnk = constant ? std::to_string(fixed.m) + ", " + std::to_string(fixed.n) + ", " +
                                           std::to_string(fixed.k)
                                     : std::string("m, n, k");
    const std::string split = constant ? std::to_string(fixed.k_split) + ", " + std::to_string(fixed.depth)
                                       : std::string("k_split, depth");
    const char* unused = constant ? "\t(void)m;\n\t(void)n;\n\t(void)k;\n" : "";
    if (!is_f32_body(body)) {
        // `a` is packed A (the graph rounds and packs it, mc_convert_pack_a_f32).
        os << "extern \"C\" __global__ void __launch_bounds__(512, 1)\n" << kGemmEpilogueKernelName
           << "(const unsigned short* __restrict__ a, const unsigned short* __restrict__ b, float* __restrict__ c, "
              "int m, int n, int k, McEpilogue epi)\n{\n"
           << unused << "\tmc_gemm16_fast<" << (body == GemmBody::Bf16Fast ? "true" : "false")
           << ", true>(a, b, c, " << mnk << ", epi);\n}\n";
        return {os.str()};
    }
    const char* bounds = body == GemmBody::F32RingBig || body == GemmBody::F32RingThin ? "256, 1"
                         : body == GemmBody::F32RingWide8                              ? "512, 1"
                         : is_narrow_body(body)                                        ? "256"
                                                                                       : "256, 2";
    os << "extern \"C\" __global__ void __launch_bounds__(" << bounds << ")\n" << kGemmEpilogueKernelName
       << "(const float* __restrict__ a, const float* __restrict__ b, float* __restrict__ c, int m, int n, int k, "
          "int k_split, int depth, float* __restrict__ partial, unsigned* __restrict__ counters, McEpilogue epi)\n{\n"
       << unused << (constant ? "\t(void)k_split;\n" : "") << "\t(void)depth;\n"
       << (folds ? "" : "\t(void)counters;\n");
    if (body == GemmBody::F32Mfma) {
        os << "\tmc_gemm_f32_mfma<true, " << (vectorized_operands ? "true" : "false") << ">(a, b, c, " << mnk
           << ", " << (constant ? std::to_string(fixed.k_split) : std::string("k_split")) << ", partial, epi);\n}\n\n";
    } else if (is_narrow_body(body)) {
        os << "\tmc_gemm_f32_narrow<" << narrow_config(body) << ">(a, b, c, "
           << mnk << ", " << split << ", partial, counters, epi);\n}\n\n";
    } else {
        const char* cfg = body == GemmBody::F32RingBig    ? "McRingBig"
                          : body == GemmBody::F32RingThin ? "McRingThin"
                          : body == GemmBody::F32RingMid  ? "McRingMid"
                          : body == GemmBody::F32RingWide8 ? "McRingWide8"
                                                          : "McRingWide";
        os << "\tmc_gemm_f32_ring<" << cfg << ">(a, b, c, "
           << mnk << ", " << split << ", partial, counters, epi);\n}\n\n";
    }
    // Split K: the partial sums added in split order (a left fold from split
    // 0's value), then the epilogue. A lane issues `chunk` split loads before
    // it adds any (indices past the last split clamped to it, their adds
    // skipped), so they are in flight together; the loads are non-temporal
    // (each partial is read once; see sum_splits_chunked).
    const int chunk = constant ? std::max(1, std::min(fixed.depth - 1, 64)) : 16;
    os << "extern \"C\" __global__ void __launch_bounds__(256)\n" << kSumSplitsEpilogueKernelName
       << "(const float* __restrict__ partial, float* __restrict__ c, unsigned count, int splits_arg, "
          "McEpilogue epi)\n{\n"
       << (constant ? "\t(void)splits_arg;\n\tconst int splits = " + std::to_string(fixed.depth) + ";\n"
                    : std::string("\tconst int splits = splits_arg;\n"))
       << "\tfor (unsigned i = blockIdx.x * 256u + threadIdx.x; i < count; i += gridDim.x * 256u) {\n"
       << "\t\tfloat s = __builtin_nontemporal_load(partial + i);\n"
       << "\t\tfor (int z0 = 1; z0 < splits; z0 += " << chunk << ") {\n"
       << "\t\t\tfloat p[" << chunk << "];\n"
       << "#pragma unroll\n"
       << "\t\t\tfor (int j = 0; j < " << chunk << "; ++j) {\n"
       << "\t\t\t\tconst int z = z0 + j < splits ? z0 + j : splits - 1;\n"
       << "\t\t\t\tp[j] = __builtin_nontemporal_load(partial + (unsigned long long)z * count + i);\n"
       << "\t\t\t}\n"
       << "#pragma unroll\n"
       << "\t\t\tfor (int j = 0; j < " << chunk << "; ++j)\n"
       << "\t\t\t\tif (z0 + j < splits) s += p[j];\n"
       << "\t\t}\n"
       << "\t\tc[i] = epi(s, i);\n\t}\n}\n";
    return {os.str()};
}

CodegenOptions codegen_options(const HipOptions& options) {
    CodegenOptions cg;
    cg.allow_vectorize = options.vectorize;
    cg.items_per_lane = options.elementwise_items;
    cg.nontemporal_loads = options.nontemporal_loads;
    cg.nontemporal_stores = options.nontemporal_stores;
    return cg;
}

FusedProgram single_op_program(OpKind op) {
    FusedProgram p;
    if (is_unary_elementwise(op)) {
        p.instrs = {FusedInstr::load(0), FusedInstr::unary(op, 0)};
    } else {
        p.instrs = {FusedInstr::load(0), FusedInstr::load(1), FusedInstr::binary(op, 0, 1)};
    }
    p.source_nodes = {op_name(op)};
    return p;
}

ElementwiseKernel generate_elementwise_kernel(const FusedProgram& program, const std::vector<Shape>& input_shapes,
                                              const Shape& out_shape, const CodegenOptions& options) {
    const std::size_t num_inputs = input_shapes.size();
    std::vector<Access> access;
    access.reserve(num_inputs);
    for (const Shape& s : input_shapes) access.push_back(classify_access(s, out_shape));

    // 16-byte vectors when the element count is a multiple of 4 and no input
    // needs per-element index math; a periodic input must repeat on a
    // vector boundary (reference rule, codegen.cpp:102-106).
    bool vec = options.allow_vectorize && num_elements(out_shape) % 4 == 0;
    for (const Access& a : access) {
        if (a.kind == Access::Kind::General) vec = false;
        if (a.kind == Access::Kind::Periodic && a.period % 4 != 0) vec = false;
    }
    const unsigned per_lane = options.items_per_lane > 0 ? options.items_per_lane : program.num_ops() >= 8 ? 8u : 4u;
    const std::string item = vec ? "mc_f32x4" : "float";

    std::ostringstream os;
    os << "// minicompiler-hip elementwise kernel: " << program.num_ops() << " op(s), out f32"
       << to_string(out_shape) << ", " << (vec ? "16-byte vector accesses" : "scalar accesses") << ", " << per_lane
       << " item(s) per lane per step.\n";
    os << "typedef float mc_f32x4 __attribute__((ext_vector_type(4)));\n\n";

    os << program_function(program, num_inputs);

    // Loads and stores.
    const std::string ld_open = options.nontemporal_loads ? "__builtin_nontemporal_load(&" : "(";
    const std::string st_prefix = options.nontemporal_stores ? "__builtin_nontemporal_store(" : "";

    os << "extern \"C\" __global__ void __launch_bounds__(" << kElementwiseBlock << ")\n"
       << kElementwiseKernelName << "(float* __restrict__ out";
    for (std::size_t k = 0; k < num_inputs; ++k) os << ", const float* __restrict__ in" << k;
    os << ", unsigned n)\n{\n";

    for (std::size_t k = 0; k < num_inputs; ++k) {
        if (access[k].kind == Access::Kind::Scalar) os << "\tconst float s" << k << " = in" << k << "[0];\n";
    }
    const std::string B = u32(kElementwiseBlock);
    const std::string step = u32(static_cast<std::size_t>(kElementwiseBlock) * per_lane);
    os << "\tconst unsigned step = gridDim.x * " << step << ";\n";
    os << "\tunsigned i = blockIdx.x * " << step << " + threadIdx.x;\n";

    // Index of item `u` of this lane for input k.
    auto index_of = [&](std::size_t k, const std::string& pos) -> std::string {
        const Access& a = access[k];
        if (a.kind == Access::Kind::Contiguous) return pos;
        if (a.kind == Access::Kind::Periodic) {
            return "(" + pos + ") % " + u32(vec ? a.period / 4 : a.period);
        }
        // General: the expression is in terms of `i`; bind it to this position.
        return "mc_general_" + std::to_string(k) + "(" + pos + ")";
    };
    std::ostringstream helpers;
    for (std::size_t k = 0; k < num_inputs; ++k) {
        if (access[k].kind == Access::Kind::General) {
            helpers << "__device__ __forceinline__ unsigned mc_general_" << k << "(unsigned i) { return "
                    << access[k].index << "; }\n";
        }
    }

    auto load_expr = [&](std::size_t k, const std::string& pos) {
        const std::string ptr = vec ? "reinterpret_cast<const mc_f32x4*>(in" + std::to_string(k) + ")"
                                    : "in" + std::to_string(k);
        return ld_open + ptr + "[" + index_of(k, pos) + "])";
    };
    // The program over one float lane of every input's item u.
    auto call = [&](const std::string& lane) {
        std::string c = "mc_program(";
        for (std::size_t k = 0; k < num_inputs; ++k) {
            if (k) c += ", ";
            c += access[k].kind == Access::Kind::Scalar ? "s" + std::to_string(k)
                                                        : "a" + std::to_string(k) + "[u]" + lane;
        }
        return c + ")";
    };
    auto store_stmt = [&](const std::string& pos, const std::string& value) {
        const std::string ptr = vec ? "reinterpret_cast<" + item + "*>(out)" : "out";
        if (options.nontemporal_stores) return st_prefix + value + ", &" + ptr + "[" + pos + "]);";
        return ptr + "[" + pos + "] = " + value + ";";
    };
    auto emit_step = [&](const std::string& indent, bool checked) {
        for (std::size_t k = 0; k < num_inputs; ++k) {
            if (access[k].kind == Access::Kind::Scalar) continue;
            os << indent << item << " a" << k << "[" << per_lane << "];\n";
        }
        os << indent << "#pragma unroll\n" << indent << "for (unsigned u = 0; u < " << per_lane << "u; ++u) {\n";
        os << indent << "\tconst unsigned p = i + u * " << B << ";\n";
        if (checked) os << indent << "\tif (p >= n) break;\n";
        for (std::size_t k = 0; k < num_inputs; ++k) {
            if (access[k].kind == Access::Kind::Scalar) continue;
            os << indent << "\ta" << k << "[u] = " << load_expr(k, "p") << ";\n";
        }
        os << indent << "}\n";
        os << indent << "#pragma unroll\n" << indent << "for (unsigned u = 0; u < " << per_lane << "u; ++u) {\n";
        os << indent << "\tconst unsigned p = i + u * " << B << ";\n";
        if (checked) os << indent << "\tif (p >= n) break;\n";
        if (vec) {
            os << indent << "\tmc_f32x4 o;\n";
            for (const char* lane : {".x", ".y", ".z", ".w"}) {
                os << indent << "\to" << lane << " = " << call(lane) << ";\n";
            }
            os << indent << "\t" << store_stmt("p", "o") << "\n";
        } else {
            os << indent << "\t" << store_stmt("p", call("")) << "\n";
        }
        // Each item's store before the next item's arithmetic, so the
        // stores go out spread over the step instead of bunched at its end.
        os << indent << "\t__builtin_amdgcn_sched_barrier(0);\n";
        os << indent << "}\n";
    };

    // Steps where all of this lane's items are in range.
    os << "\tfor (; i + " << u32(static_cast<std::size_t>(kElementwiseBlock) * (per_lane - 1)) << " < n; i += step) {\n";
    emit_step("\t\t", false);
    os << "\t}\n";
    // At most one ragged step remains for this lane.
    os << "\tif (i < n) {\n";
    emit_step("\t\t", true);
    os << "\t}\n}\n";

    // General-access index helpers go in front of the kernel.
    std::string text = os.str();
    if (!helpers.str().empty()) {
        const std::size_t kernel_at = text.find("extern \"C\" __global__");
        text.insert(kernel_at, helpers.str() + "\n");
    }
    ElementwiseKernel k;
    k.source = std::move(text);
    k.vectorized = vec;
    k.items_per_lane = per_lane;
    return k;
}

}  // namespace minicompiler::hip
