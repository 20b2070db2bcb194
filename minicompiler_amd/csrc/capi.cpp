// The C ABI (include/minicompiler_hip.h). Part 1 keeps the reference's
// bench/capi.cpp:62-235 contract; part 2 is this backend's additions.

#include "minicompiler_hip.h"

#include "hip/codegen.hpp"
#include "hip/rtc_sources.hpp"
#include "hip/hip_rt.h"
#include "hip/kernel_compiler.hpp"
#include "hip/matmul.h"
#include "hip/matmul_policy.hpp"
#include "minicompiler/hip/hip_backend.hpp"
#include "minicompiler/parser.hpp"
#include "minicompiler/passes/pipeline.hpp"
#include "minicompiler/random.hpp"
#include "minicompiler/runtime/memory_plan.hpp"

#include <cerrno>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <memory>
#include <sstream>
#include <string>
#include <vector>

using namespace minicompiler;

namespace {

thread_local std::string g_last_error;

int fail(const std::string& message) {
    g_last_error = message;
    return 1;
}

struct StageStats {
    std::string pass;
    GraphStats stats;
};

struct Compiled {
    Graph graph;
    std::vector<StageStats> stages;
    hip::HipOptions options;
    std::unique_ptr<hip::HipExecutable> exe;  // null for backend "none"
    std::vector<const float*> inputs;
    std::vector<float*> outputs;
    // Profiling events: steps x (launches + 1).
    std::vector<void*> events;
    int profile_steps = 0;
    int profile_used = 0;

    void release_events() {
        for (void* e : events) mchip_event_destroy(e);
        events.clear();
        profile_steps = profile_used = 0;
    }
    ~Compiled() { release_events(); }
};

Compiled* as_compiled(void* h) { return static_cast<Compiled*>(h); }
const Compiled* as_compiled(const void* h) { return static_cast<const Compiled*>(h); }

int copy_text(char* out, int size, const std::string& text) {
    if (out && size > 0) std::snprintf(out, static_cast<std::size_t>(size), "%s", text.c_str());
    return static_cast<int>(text.size());
}

void write_error(char* error, int size, const std::string& message) {
    g_last_error = message;
    copy_text(error, size, message);
}

Result<std::map<std::string, std::string>> split_pairs(const char* spec, const char* what) {
    std::map<std::string, std::string> out;
    std::stringstream list(spec ? spec : "");
    for (std::string item; std::getline(list, item, ',');) {
        if (item.empty()) continue;
        const std::size_t eq = item.find('=');
        if (eq == std::string::npos || eq == 0) {
            return Error{std::string("bad ") + what + " '" + item + "', expected NAME=VALUE"};
        }
        out[item.substr(0, eq)] = item.substr(eq + 1);
    }
    return out;
}

Result<long long> to_integer(const std::string& s) {
    char* end = nullptr;
    errno = 0;
    const long long v = std::strtoll(s.c_str(), &end, 10);
    if (s.empty() || *end != '\0' || errno == ERANGE) return Error{"expected an integer, got '" + s + "'"};
    return v;
}

Result<hip::HipOptions> parse_options(const char* spec) {
    auto pairs = split_pairs(spec, "option");
    if (!pairs.ok()) return pairs.error();
    hip::HipOptions o;
    for (const auto& [key, value] : pairs.value()) {
        if (key == "matmul") {
            Result<hip::MatmulKernel> k = hip::matmul_kernel_from_name(value);
            if (!k.ok()) return k.error();
            o.matmul = k.value();
        } else if (key == "vectorize") {
            o.vectorize = value != "0" && value != "false";
        } else if (key == "device") {
            Result<long long> d = to_integer(value);
            if (!d.ok()) return d.error();
            o.device = static_cast<int>(d.value());
        } else if (key == "ew_items" || key == "ew_blocks_per_cu") {
            Result<long long> v = to_integer(value);
            if (!v.ok()) return v.error();
            if (v.value() < 0 || v.value() > 64) {
                return Error{"option " + key + " out of range: " + value};
            }
            (key == "ew_items" ? o.elementwise_items : o.elementwise_blocks_per_cu) = static_cast<unsigned>(v.value());
        } else if (key == "tc_convert") {
            o.convert_tensor_core_operands = value != "0" && value != "false";
        } else if (key == "epilogue") {
            o.fuse_epilogue = value != "0" && value != "false";
        } else if (key == "graph") {
            o.graph_replay = value != "0" && value != "false";
        } else if (key == "autotune") {
            o.autotune = value != "0" && value != "false";
        } else if (key == "split_fold") {
            o.split_fold = value != "0" && value != "false";
        } else if (key == "ring") {
            static const char* const names[] = {"auto", "wide", "mid", "big", "thin", "narrow", "wide8"};
            int cfg = -1;
            for (int i = 0; i < 7; ++i) {
                if (value == names[i]) cfg = i;
            }
            if (cfg < 0) {
                return Error{"option ring=" + value + ": expected auto, wide, wide8, mid, big, thin or narrow"};
            }
            o.ring_config = cfg;
        } else if (key == "ew_nt_loads") {
            o.nontemporal_loads = value != "0" && value != "false";
        } else if (key == "ew_nt_stores") {
            o.nontemporal_stores = value != "0" && value != "false";
        } else {
            return Error{"unknown option '" + key +
                         "' (matmul, vectorize, device, epilogue, graph, autotune, split_fold, ring, tc_convert, "
                         "ew_items, ew_nt_loads, ew_nt_stores, ew_blocks_per_cu)"};
        }
    }
    return o;
}

void* compile_graph(Result<Graph> parsed, const char* passes, const char* backend, const char* options, char* error,
                    int error_size) {
    if (!parsed.ok()) {
        write_error(error, error_size, parsed.error().message);
        return nullptr;
    }
    Result<std::vector<std::string>> pipeline = parse_pipeline(passes ? passes : "default");
    if (!pipeline.ok()) {
        write_error(error, error_size, pipeline.error().message);
        return nullptr;
    }
    auto c = std::make_unique<Compiled>();
    Result<Graph> optimized = run_pipeline(parsed.value(), pipeline.value(), nullptr,
                                           [&](std::size_t, const std::string& pass, const Graph& g) {
                                               c->stages.push_back({pass, compute_stats(g)});
                                           });
    if (!optimized.ok()) {
        write_error(error, error_size, optimized.error().message);
        return nullptr;
    }
    c->graph = std::move(optimized).value();
    Result<hip::HipOptions> opts = parse_options(options);
    if (!opts.ok()) {
        write_error(error, error_size, opts.error().message);
        return nullptr;
    }
    c->options = opts.value();
    const std::string b = backend ? backend : "hip";
    if (b == "hip") {
        Result<std::unique_ptr<hip::HipExecutable>> exe = hip::compile_for_hip(c->graph, c->options);
        if (!exe.ok()) {
            write_error(error, error_size, exe.error().message);
            return nullptr;
        }
        c->exe = std::move(exe).value();
    } else if (b != "none") {
        Result<std::unique_ptr<Backend>> unknown = create_backend(b);
        write_error(error, error_size,
                    unknown.ok() ? "backend '" + b + "' has no executable here" : unknown.error().message);
        return nullptr;
    }
    return c.release();
}

Result<ParseOptions> parse_dims(const char* dims) {
    auto pairs = split_pairs(dims, "dim");
    if (!pairs.ok()) return pairs.error();
    ParseOptions o;
    for (const auto& [key, value] : pairs.value()) {
        Result<long long> v = to_integer(value);
        if (!v.ok()) return Error{"bad dim '" + key + "=" + value + "', expected NAME=VALUE"};
        o.dims[key] = v.value();
    }
    return o;
}

// Minimal JSON text helpers.
std::string quote(const std::string& s) {
    std::string o = "\"";
    for (char ch : s) {
        if (ch == '"' || ch == '\\') {
            o += '\\';
            o += ch;
        } else if (static_cast<unsigned char>(ch) < 0x20) {
            char buf[8];
            std::snprintf(buf, sizeof buf, "\\u%04x", ch);
            o += buf;
        } else {
            o += ch;
        }
    }
    return o + "\"";
}

std::string json_shape(const Shape& s) {
    std::string o = "[";
    for (std::size_t i = 0; i < s.size(); ++i) o += (i ? "," : "") + std::to_string(s[i]);
    return o + "]";
}

std::string json_ids(const std::vector<NodeId>& ids) {
    std::string o = "[";
    for (std::size_t i = 0; i < ids.size(); ++i) o += (i ? "," : "") + std::to_string(ids[i]);
    return o + "]";
}

std::string json_stats(const GraphStats& s) {
    std::ostringstream o;
    o << "{\"nodes\":" << s.nodes << ",\"inputs\":" << s.inputs << ",\"constants\":" << s.constants
      << ",\"compute_nodes\":" << s.compute_nodes << ",\"fused_nodes\":" << s.fused_nodes
      << ",\"elementwise_ops\":" << s.elementwise_ops << ",\"matmuls\":" << s.matmuls << "}";
    return o.str();
}

std::string json_program(const FusedProgram& p) {
    std::ostringstream o;
    o << "[";
    for (std::size_t r = 0; r < p.instrs.size(); ++r) {
        const FusedInstr& ins = p.instrs[r];
        std::uint32_t bits = 0;
        std::memcpy(&bits, &ins.immediate, 4);
        o << (r ? "," : "") << "{\"kind\":" << static_cast<int>(ins.kind) << ",\"op\":" << static_cast<int>(ins.op)
          << ",\"a\":" << ins.a << ",\"b\":" << ins.b << ",\"imm_bits\":" << bits << "}";
    }
    o << "]";
    return o.str();
}

std::string graph_json(const Graph& g) {
    std::ostringstream o;
    o << "{\"name\":" << quote(g.name()) << ",\"nodes\":[";
    for (std::size_t i = 0; i < g.num_nodes(); ++i) {
        const Node& n = g.node(static_cast<NodeId>(i));
        o << (i ? "," : "") << "{\"id\":" << i << ",\"op\":" << static_cast<int>(n.op) << ",\"op_name\":"
          << quote(op_name(n.op)) << ",\"name\":" << quote(n.name) << ",\"inputs\":" << json_ids(n.inputs)
          << ",\"shape\":" << json_shape(n.type.shape);
        if (n.op == OpKind::FusedElementwise) {
            o << ",\"program\":" << json_program(*n.fused) << ",\"sources\":[";
            for (std::size_t k = 0; k < n.fused->source_nodes.size(); ++k) {
                o << (k ? "," : "") << quote(n.fused->source_nodes[k]);
            }
            o << "]";
        }
        o << "}";
    }
    o << "],\"inputs\":" << json_ids(g.inputs()) << ",\"outputs\":" << json_ids(g.outputs()) << "}";
    return o.str();
}

// "r3 = mul r1, r2" lines; immediates as decimal or 0x bit patterns.
Result<FusedProgram> parse_program(const std::string& text) {
    FusedProgram p;
    std::istringstream in(text);
    for (std::string line; std::getline(in, line);) {
        const std::size_t eq = line.find('=');
        if (line.find_first_not_of(" \t\r") == std::string::npos) continue;
        if (eq == std::string::npos) return Error{"bad program line '" + line + "'"};
        std::istringstream rhs(line.substr(eq + 1));
        std::string word;
        rhs >> word;
        auto reg = [](std::string t) -> Result<std::int32_t> {
            if (!t.empty() && t.back() == ',') t.pop_back();
            if (t.size() < 2 || (t[0] != 'r' && t.rfind("in", 0) != 0)) return Error{"bad operand '" + t + "'"};
            Result<long long> v = to_integer(t.substr(t[0] == 'r' ? 1 : 2));
            if (!v.ok()) return v.error();
            return static_cast<std::int32_t>(v.value());
        };
        if (word == "load") {
            std::string a;
            rhs >> a;
            Result<std::int32_t> r = reg(a);
            if (!r.ok()) return r.error();
            p.instrs.push_back(FusedInstr::load(r.value()));
        } else if (word == "imm") {
            std::string v;
            rhs >> v;
            float f = 0.0f;
            if (v.rfind("0x", 0) == 0) {
                const auto bits = static_cast<std::uint32_t>(std::strtoul(v.c_str(), nullptr, 16));
                std::memcpy(&f, &bits, 4);
            } else {
                f = std::strtof(v.c_str(), nullptr);
            }
            p.instrs.push_back(FusedInstr::imm(f));
        } else {
            const std::optional<OpKind> op = op_from_name(word);
            if (!op || !is_elementwise(*op)) return Error{"unknown op '" + word + "'"};
            std::string a, b;
            rhs >> a >> b;
            Result<std::int32_t> ra = reg(a);
            if (!ra.ok()) return ra.error();
            if (is_unary_elementwise(*op)) {
                p.instrs.push_back(FusedInstr::unary(*op, ra.value()));
            } else {
                Result<std::int32_t> rb = reg(b);
                if (!rb.ok()) return rb.error();
                p.instrs.push_back(FusedInstr::binary(*op, ra.value(), rb.value()));
            }
        }
    }
    return p;
}

Result<Shape> parse_shape(const std::string& text) {
    const std::size_t l = text.find('['), r = text.rfind(']');
    if (l == std::string::npos || r == std::string::npos || r < l) return Error{"bad shape '" + text + "'"};
    Shape s;
    std::stringstream dims(text.substr(l + 1, r - l - 1));
    for (std::string d; std::getline(dims, d, ',');) {
        if (d.find_first_not_of(" ") == std::string::npos) continue;
        Result<long long> v = to_integer(d.substr(d.find_first_not_of(" ")));
        if (!v.ok()) return v.error();
        s.push_back(v.value());
    }
    return s;
}

}  // namespace

extern "C" {

// ---------------------------------------------------------------- part 1

MC_API void* mc_compile(const char* graph_path, const char* dims, const char* passes, const char* backend,
                        char* error, int error_size) {
    Result<ParseOptions> options = parse_dims(dims);
    if (!options.ok()) {
        write_error(error, error_size, options.error().message);
        return nullptr;
    }
    return compile_graph(parse_graph_file(graph_path ? graph_path : "", options.value()), passes, backend, nullptr,
                         error, error_size);
}

MC_API int mc_num_inputs(const void* h) { return static_cast<int>(as_compiled(h)->graph.inputs().size()); }
MC_API int mc_num_outputs(const void* h) { return static_cast<int>(as_compiled(h)->graph.outputs().size()); }

MC_API long long mc_output_elements(const void* h, int k) {
    const Graph& g = as_compiled(h)->graph;
    if (k < 0 || static_cast<std::size_t>(k) >= g.outputs().size()) return -1;
    return static_cast<long long>(g.node(g.outputs()[static_cast<std::size_t>(k)]).type.num_elements());
}

MC_API int mc_run(void* h, const float* const* inputs, float* const* outputs) {
    Compiled* c = as_compiled(h);
    if (!c->exe) return fail("mc_run: compiled without an executable (backend \"none\")");
    c->inputs.assign(inputs, inputs + c->graph.inputs().size());
    c->outputs.assign(outputs, outputs + c->graph.outputs().size());
    Status st = c->exe->run_buffers(c->inputs, c->outputs);
    return st.ok() ? 0 : fail(st.message());
}

MC_API int mc_upload(void* h, const float* const* inputs) {
    Compiled* c = as_compiled(h);
    if (!c->exe) return fail("mc_upload: no executable");
    c->inputs.assign(inputs, inputs + c->graph.inputs().size());
    Status st = c->exe->upload_inputs(c->inputs);
    if (st.ok()) st = c->exe->synchronize();
    return st.ok() ? 0 : fail(st.message());
}

MC_API int mc_enqueue(void* h, void* stream) {
    Compiled* c = as_compiled(h);
    if (!c->exe) return fail("mc_enqueue: no executable");
    Status st = c->exe->enqueue(stream);
    return st.ok() ? 0 : fail(st.message());
}

MC_API int mc_launch_nodes(void* h, char* out, int size) {
    const Compiled* c = as_compiled(h);
    if (!c->exe) return fail("mc_launch_nodes: no executable");
    std::string text;
    for (const std::vector<NodeId>& ids : c->exe->launch_nodes()) {
        if (!text.empty()) text += ';';
        for (std::size_t k = 0; k < ids.size(); ++k) text += (k ? "," : "") + std::to_string(ids[k]);
    }
    return copy_text(out, size, text);
}

MC_API int mc_enqueue_launch(void* h, int j, void* stream) {
    Compiled* c = as_compiled(h);
    if (!c->exe) return fail("mc_enqueue_launch: no executable");
    if (j < 0) return fail("mc_enqueue_launch: negative launch index");
    Status st = c->exe->enqueue_launch(static_cast<std::size_t>(j), stream);
    return st.ok() ? 0 : fail(st.message());
}

MC_API int mc_enqueue_steps(void* h, int launch, int steps, int sets, const void* const* set_inputs,
                            void* const* set_outputs, void* stream, double* host_us_per_step) {
    Compiled* c = as_compiled(h);
    if (!c->exe) return fail("mc_enqueue_steps: no executable");
    if (steps < 0 || sets < 0 || (sets > 0 && (set_inputs == nullptr || set_outputs == nullptr))) {
        return fail("mc_enqueue_steps: bad step or buffer-set arguments");
    }
    if (launch >= static_cast<int>(c->exe->kernel_launches())) {
        return fail("mc_enqueue_steps: launch " + std::to_string(launch) + " out of range");
    }
    const std::size_t ni = c->graph.inputs().size(), no = c->graph.outputs().size();
    // The sets' pointers, built once: binding a set then only copies them in.
    std::vector<std::vector<const void*>> ins(static_cast<std::size_t>(sets));
    std::vector<std::vector<void*>> outs(static_cast<std::size_t>(sets));
    for (int r = 0; r < sets; ++r) {
        ins[r].assign(set_inputs + static_cast<std::size_t>(r) * ni, set_inputs + (static_cast<std::size_t>(r) + 1) * ni);
        outs[r].assign(set_outputs + static_cast<std::size_t>(r) * no,
                       set_outputs + (static_cast<std::size_t>(r) + 1) * no);
    }
    const auto t0 = std::chrono::steady_clock::now();
    if (sets == 0 && launch < 0) {
        // Every step on the same buffers: one call (graph_replay replays
        // runs of captured steps).
        Status st = c->exe->enqueue_steps(steps, stream);
        if (!st.ok()) return fail("mc_enqueue_steps: " + st.message());
    }
    for (int i = 0; i < steps && (sets > 0 || launch >= 0); ++i) {
        if (sets > 0) {
            const std::size_t r = static_cast<std::size_t>(i % sets);
            Status st = c->exe->bind_inputs(ins[r]);
            if (st.ok()) st = c->exe->bind_outputs(outs[r]);
            if (!st.ok()) return fail("mc_enqueue_steps: " + st.message());
        }
        Status st = launch < 0 ? c->exe->enqueue(stream) : c->exe->enqueue_launch(static_cast<std::size_t>(launch), stream);
        if (!st.ok()) return fail("mc_enqueue_steps: " + st.message());
    }
    if (host_us_per_step) {
        const double us = std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count();
        *host_us_per_step = steps > 0 ? us / steps : 0.0;
    }
    return 0;
}

MC_API int mc_download(void* h, float* const* outputs) {
    Compiled* c = as_compiled(h);
    if (!c->exe) return fail("mc_download: no executable");
    c->outputs.assign(outputs, outputs + c->graph.outputs().size());
    Status st = c->exe->download_outputs(c->outputs);
    return st.ok() ? 0 : fail(st.message());
}

MC_API int mc_kernel_launches(void* h) {
    const Compiled* c = as_compiled(h);
    return c->exe ? static_cast<int>(c->exe->kernel_launches()) : -1;
}

MC_API int mc_matmul_kernels(void* h, char* out, int size) {
    const Compiled* c = as_compiled(h);
    if (!c->exe) return fail("mc_matmul_kernels: no executable");
    std::string names;
    for (hip::MatmulKernel k : c->exe->matmul_kernels()) names += (names.empty() ? "" : ",") + std::string(hip::matmul_kernel_name(k));
    copy_text(out, size, names);
    return 0;
}

MC_API double mc_gpu_sm_clock_mhz(void) { return hip::current_clock_mhz(0); }

MC_API int mc_gpu_clock_sample(double* mhz, unsigned long long* stamp_ns) {
    double v = 0.0;
    unsigned long long t = 0;
    const bool ok = hip::current_clock_sample(0, &v, &t);
    if (mhz) *mhz = v;
    if (stamp_ns) *stamp_ns = t;
    return ok ? 0 : 1;
}

MC_API int mc_gpu_device_json(const double* clocks, int n, char* out, int size) {
    Result<hip::DeviceInfo> d = hip::query_device(0);
    if (!d.ok()) return 1;
    const hip::DeviceInfo& i = d.value();
    double lo = 0, hi = 0, mean = 0;
    const int count = clocks ? n : 0;
    for (int j = 0; j < count; ++j) {
        lo = j ? std::min(lo, clocks[j]) : clocks[j];
        hi = j ? std::max(hi, clocks[j]) : clocks[j];
        mean += clocks[j] / count;
    }
    std::ostringstream o;
    o.precision(10);
    o << "{\"name\":" << quote(i.name) << ",\"arch\":" << quote(i.arch) << ",\"cu_count\":" << i.cu_count
      << ",\"wave_size\":" << i.wave_size << ",\"clock_mhz\":" << i.clock_mhz << ",\"mem_clock_mhz\":" << i.mem_clock_mhz
      << ",\"bus_width_bits\":" << i.bus_width_bits << ",\"total_memory\":" << i.total_memory
      << ",\"l2_bytes\":" << i.l2_bytes << ",\"lds_bytes_per_block\":" << i.lds_bytes_per_block
      << ",\"runtime_version\":" << i.runtime_version << ",\"driver_version\":" << i.driver_version
      << ",\"peak_bandwidth_gbs\":" << i.peak_bandwidth_gbs() << ",\"peak_fp32_gflops\":" << i.peak_fp32_gflops(i.clock_mhz)
      << ",\"peak_bf16_gflops\":" << i.peak_bf16_gflops(i.clock_mhz)
      << ",\"clock_now_mhz\":" << hip::current_clock_mhz(0) << ",\"clocks\":{\"samples\":" << count
      << ",\"min_mhz\":" << lo << ",\"max_mhz\":" << hi << ",\"mean_mhz\":" << mean << "}}";
    const std::string text = o.str();
    if (static_cast<int>(text.size()) >= size) return 2;
    copy_text(out, size, text);
    return 0;
}

MC_API void mc_release(void* h) { delete as_compiled(h); }

// ---------------------------------------------------------------- part 2

MC_API void* mc_compile_source(const char* text, const char* dims, const char* passes, const char* backend,
                               const char* options, char* error, int error_size) {
    Result<ParseOptions> parse_options = parse_dims(dims);
    if (!parse_options.ok()) {
        write_error(error, error_size, parse_options.error().message);
        return nullptr;
    }
    return compile_graph(parse_graph(text ? text : "", parse_options.value()), passes, backend, options, error,
                         error_size);
}

MC_API int mc_last_error(char* out, int size) { return copy_text(out, size, g_last_error); }

MC_API long long mc_input_elements(const void* h, int k) {
    const Graph& g = as_compiled(h)->graph;
    if (k < 0 || static_cast<std::size_t>(k) >= g.inputs().size()) return -1;
    return static_cast<long long>(g.node(g.inputs()[static_cast<std::size_t>(k)]).type.num_elements());
}

MC_API int mc_bind_inputs(void* h, const void* const* device_inputs) {
    Compiled* c = as_compiled(h);
    if (!c->exe) return fail("mc_bind_inputs: no executable");
    std::vector<const void*> v(device_inputs, device_inputs + c->graph.inputs().size());
    Status st = c->exe->bind_inputs(v);
    return st.ok() ? 0 : fail(st.message());
}

MC_API int mc_bind_outputs(void* h, void* const* device_outputs) {
    Compiled* c = as_compiled(h);
    if (!c->exe) return fail("mc_bind_outputs: no executable");
    std::vector<void*> v(device_outputs, device_outputs + c->graph.outputs().size());
    Status st = c->exe->bind_outputs(v);
    return st.ok() ? 0 : fail(st.message());
}

MC_API void* mc_input_device_ptr(void* h, int k) {
    Compiled* c = as_compiled(h);
    return c->exe && k >= 0 ? c->exe->input_device_ptr(static_cast<std::size_t>(k)) : nullptr;
}

MC_API void* mc_output_device_ptr(void* h, int k) {
    Compiled* c = as_compiled(h);
    return c->exe && k >= 0 ? c->exe->output_device_ptr(static_cast<std::size_t>(k)) : nullptr;
}

MC_API void* mc_stream(void* h) {
    Compiled* c = as_compiled(h);
    return c->exe ? c->exe->stream() : nullptr;
}

MC_API int mc_synchronize(void* h) {
    Compiled* c = as_compiled(h);
    if (!c->exe) return fail("mc_synchronize: no executable");
    Status st = c->exe->synchronize();
    return st.ok() ? 0 : fail(st.message());
}

MC_API double mc_jit_compile_ms(void* h) {
    const Compiled* c = as_compiled(h);
    return c->exe ? c->exe->jit_compile_ms() : 0.0;
}

MC_API long long mc_intermediate_bytes(void* h) {
    const Compiled* c = as_compiled(h);
    return c->exe ? static_cast<long long>(c->exe->intermediate_bytes())
                  : static_cast<long long>(plan_memory(c->graph).bytes_with_reuse());
}

MC_API long long mc_arena_bytes(void* h) {
    const Compiled* c = as_compiled(h);
    return c->exe ? static_cast<long long>(c->exe->arena_bytes()) : 0;
}

MC_API int mc_profile_start(void* h, int steps) {
    Compiled* c = as_compiled(h);
    if (!c->exe) return fail("mc_profile_start: no executable");
    if (steps < 1) return fail("mc_profile_start: steps must be >= 1");
    c->release_events();
    const std::size_t per = c->exe->kernel_launches() + 1;
    for (std::size_t i = 0; i < per * static_cast<std::size_t>(steps); ++i) {
        void* e = nullptr;
        const int rc = mchip_event_create(&e);
        if (rc != 0) {
            c->release_events();
            return fail(std::string("hipEventCreate: ") + mchip_error_string(rc));
        }
        c->events.push_back(e);
    }
    c->profile_steps = steps;
    return 0;
}

MC_API int mc_enqueue_profiled(void* h, void* stream) {
    Compiled* c = as_compiled(h);
    if (!c->exe) return fail("mc_enqueue_profiled: no executable");
    if (c->profile_used >= c->profile_steps) return fail("mc_enqueue_profiled: no profile slots left");
    const std::size_t per = c->exe->kernel_launches() + 1;
    Status st = c->exe->enqueue_with_events(stream, c->events.data() + per * static_cast<std::size_t>(c->profile_used));
    if (!st.ok()) return fail(st.message());
    ++c->profile_used;
    return 0;
}

MC_API int mc_profile_read(void* h, float* ms, int capacity) {
    Compiled* c = as_compiled(h);
    if (!c->exe) return fail("mc_profile_read: no executable"), -1;
    const std::size_t launches = c->exe->kernel_launches();
    const std::size_t per = launches + 1;
    int written = 0;
    for (int s = 0; s < c->profile_used; ++s) {
        void* const* ev = c->events.data() + per * static_cast<std::size_t>(s);
        int rc = mchip_event_synchronize(ev[launches]);
        if (rc != 0) return fail(std::string("hipEventSynchronize: ") + mchip_error_string(rc)), -1;
        for (std::size_t j = 0; j < launches; ++j) {
            float t = 0.0f;
            rc = mchip_event_elapsed_ms(&t, ev[j], ev[j + 1]);
            if (rc != 0) return fail(std::string("hipEventElapsedTime: ") + mchip_error_string(rc)), -1;
            if (written < capacity) ms[written] = t;
            ++written;
        }
    }
    return written;
}

MC_API int mc_launch_names(void* h, char* out, int size) {
    const Compiled* c = as_compiled(h);
    if (!c->exe) return fail("mc_launch_names: no executable"), -1;
    std::string all;
    for (const std::string& n : c->exe->launch_names()) all += n + "\n";
    return copy_text(out, size, all);
}

MC_API void mc_fill_uniform(float* out, size_t count, unsigned long long seed, float lo, float hi) {
    fill_uniform(out, count, seed, lo, hi);
}

MC_API void mc_fill_normal(float* out, size_t count, unsigned long long seed, double mean, double stddev) {
    fill_normal(out, count, seed, mean, stddev);
}

MC_API int mc_graph_json(const void* h, char* out, int size) { return copy_text(out, size, graph_json(as_compiled(h)->graph)); }

MC_API int mc_constant_values(const void* h, int node, float* out, long long count) {
    const Graph& g = as_compiled(h)->graph;
    if (node < 0 || static_cast<std::size_t>(node) >= g.num_nodes()) return fail("no node " + std::to_string(node));
    const Node& n = g.node(node);
    if (n.op != OpKind::Constant) return fail("node " + std::to_string(node) + " is not a constant");
    if (count != static_cast<long long>(n.constant->size())) return fail("wrong element count for constant");
    std::memcpy(out, n.constant->data(), n.constant->size() * sizeof(float));
    return 0;
}

MC_API int mc_stage_stats_json(const void* h, char* out, int size) {
    const Compiled* c = as_compiled(h);
    std::string o = "[";
    for (std::size_t i = 0; i < c->stages.size(); ++i) {
        o += (i ? "," : "") + std::string("{\"pass\":") + quote(c->stages[i].pass) + ",\"stats\":" +
             json_stats(c->stages[i].stats) + "}";
    }
    return copy_text(out, size, o + "]");
}

MC_API int mc_plan_json(const void* h, int pool_outputs, char* out, int size) {
    PlanOptions po;
    po.pool_outputs = pool_outputs != 0;
    const MemoryPlan p = plan_memory(as_compiled(h)->graph, po);
    std::ostringstream o;
    o << "{\"buffer_of\":[";
    for (std::size_t i = 0; i < p.buffer_of.size(); ++i) o << (i ? "," : "") << p.buffer_of[i];
    o << "],\"buffer_bytes\":[";
    for (std::size_t i = 0; i < p.buffer_bytes.size(); ++i) o << (i ? "," : "") << p.buffer_bytes[i];
    o << "],\"last_use\":[";
    for (std::size_t i = 0; i < p.last_use.size(); ++i) o << (i ? "," : "") << p.last_use[i];
    o << "],\"bytes_without_reuse\":" << p.bytes_without_reuse << ",\"bytes_with_reuse\":" << p.bytes_with_reuse() << "}";
    return copy_text(out, size, o.str());
}

MC_API int mc_kernel_sources(const void* h, char* out, int size) {
    const Compiled* c = as_compiled(h);
    std::vector<std::string> sources;
    if (c->exe) {
        sources = c->exe->kernel_sources();
    } else {
        const hip::CodegenOptions cg = hip::codegen_options(c->options);
        for (const Node& n : c->graph.nodes()) {
            if (!is_elementwise(n.op) && n.op != OpKind::FusedElementwise) continue;
            const FusedProgram p = n.op == OpKind::FusedElementwise ? *n.fused : hip::single_op_program(n.op);
            std::vector<Shape> shapes;
            for (NodeId in : n.inputs) shapes.push_back(c->graph.node(in).type.shape);
            sources.push_back(hip::generate_elementwise_kernel(p, shapes, n.type.shape, cg).source);
        }
    }
    std::string all;
    for (std::size_t i = 0; i < sources.size(); ++i) all += (i ? "//----\n" : "") + sources[i];
    return copy_text(out, size, all);
}

MC_API int mc_print_graph(const void* h, char* out, int size) { return copy_text(out, size, print_graph(as_compiled(h)->graph)); }

MC_API int mc_generate_elementwise_kernel(const char* program, const char* input_shapes, const char* out_shape,
                                          int allow_vectorize, int items_per_lane, int* vectorized, char* out,
                                          int size) {
    Result<FusedProgram> p = parse_program(program ? program : "");
    if (!p.ok()) return fail(p.error().message), -1;
    std::vector<Shape> shapes;
    std::stringstream list(input_shapes ? input_shapes : "");
    for (std::string item; std::getline(list, item, ';');) {
        if (item.find('[') == std::string::npos) continue;
        Result<Shape> s = parse_shape(item);
        if (!s.ok()) return fail(s.error().message), -1;
        shapes.push_back(s.value());
    }
    Result<Shape> os = parse_shape(out_shape ? out_shape : "");
    if (!os.ok()) return fail(os.error().message), -1;
    Status st = validate(p.value(), shapes.size());
    if (!st.ok()) return fail(st.message()), -1;
    hip::CodegenOptions cg;
    cg.allow_vectorize = allow_vectorize != 0;
    if (items_per_lane > 0) cg.items_per_lane = static_cast<unsigned>(items_per_lane);
    const hip::ElementwiseKernel k = hip::generate_elementwise_kernel(p.value(), shapes, os.value(), cg);
    if (vectorized) *vectorized = k.vectorized ? 1 : 0;
    return copy_text(out, size, k.source);
}

MC_API int mc_generate_gemm_epilogue_kernel(const char* program, int acc_input, const char* input_shapes,
                                            const char* out_shape, int vectorized_operands, const char* body,
                                            char* out, int size) {
    struct BodyName {
        const char* name;
        hip::GemmBody body;
        const char* const* source;
    };
    static const BodyName kBodies[] = {
        {"two_stage", hip::GemmBody::F32Mfma, &hip::kGemmF32MfmaSource},
        {"ring_big", hip::GemmBody::F32RingBig, &hip::kGemmF32RingSource},
        {"ring_wide", hip::GemmBody::F32RingWide, &hip::kGemmF32RingSource},
        {"ring_wide8", hip::GemmBody::F32RingWide8, &hip::kGemmF32RingSource},
        {"ring_mid", hip::GemmBody::F32RingMid, &hip::kGemmF32RingSource},
        {"ring_thin", hip::GemmBody::F32RingThin, &hip::kGemmF32RingSource},
        {"narrow16", hip::GemmBody::F32Narrow16, &hip::kGemmF32NarrowSource},
        {"narrow32", hip::GemmBody::F32Narrow32, &hip::kGemmF32NarrowSource},
        {"narrow16x64", hip::GemmBody::F32Narrow16x64, &hip::kGemmF32NarrowSource},
        {"narrow16x32", hip::GemmBody::F32Narrow16x32, &hip::kGemmF32NarrowSource},
        {"narrow64", hip::GemmBody::F32Narrow64, &hip::kGemmF32NarrowSource},
        {"bf16", hip::GemmBody::Bf16Fast, &hip::kGemm16FastSource},
        {"f16", hip::GemmBody::F16Fast, &hip::kGemm16FastSource},
    };
    const BodyName* chosen = nullptr;
    const std::string want = body && *body ? body : "two_stage";
    for (const BodyName& b : kBodies) {
        if (want == b.name) chosen = &b;
    }
    if (chosen == nullptr) return fail("mc_generate_gemm_epilogue_kernel: unknown body '" + want + "'"), -1;
    Result<FusedProgram> p = parse_program(program ? program : "");
    if (!p.ok()) return fail(p.error().message), -1;
    std::vector<Shape> shapes;
    std::stringstream list(input_shapes ? input_shapes : "");
    for (std::string item; std::getline(list, item, ';');) {
        if (item.find('[') == std::string::npos) continue;
        Result<Shape> s = parse_shape(item);
        if (!s.ok()) return fail(s.error().message), -1;
        shapes.push_back(s.value());
    }
    Result<Shape> os = parse_shape(out_shape ? out_shape : "");
    if (!os.ok()) return fail(os.error().message), -1;
    Status st = validate(p.value(), shapes.size());
    if (!st.ok()) return fail(st.message()), -1;
    if (acc_input < 0 || static_cast<std::size_t>(acc_input) >= shapes.size()) {
        return fail("mc_generate_gemm_epilogue_kernel: acc_input out of range"), -1;
    }
    const hip::GemmEpilogueKernel k = hip::generate_gemm_epilogue_kernel(
        p.value(), static_cast<std::size_t>(acc_input), shapes, os.value(), vectorized_operands != 0,
        *chosen->source, chosen->body);
    return copy_text(out, size, k.source);
}

MC_API int mc_compile_kernel_source(const char* source, const char* arch, char* log, int log_size) {
    Result<std::string> code = hip::KernelCompiler::compile_code_object(source ? source : "", arch ? arch : "gfx950");
    if (!code.ok()) {
        copy_text(log, log_size, code.error().message);
        return fail(code.error().message);
    }
    copy_text(log, log_size, "");
    return 0;
}

MC_API int mc_launch_matmul(int kernel, const float* a, const float* b, float* c, int m, int n, int k, void* stream,
                            int splits, float* workspace) {
    return mchip_launch_matmul(kernel, a, b, c, m, n, k, stream, splits, workspace);
}

MC_API int mc_launch_matmul_cfg(int kernel, const float* a, const float* b, float* c, int m, int n, int k,
                                void* stream, int splits, float* workspace, int ring_cfg) {
    return mchip_launch_matmul_cfg(kernel, a, b, c, m, n, k, stream, splits, workspace, ring_cfg);
}

MC_API int mc_launch_matmul_noalloc(int kernel, const float* a, const float* b, float* c, int m, int n, int k,
                                    void* stream, int splits) {
    const unsigned long long need = mchip_noalloc_required_bytes(kernel, m, n, splits);
    const unsigned long long have = mchip_noalloc_scratch_bytes();
    if (need > have) {
        g_last_error = "mc_launch_matmul_noalloc: " + std::to_string(splits) + " splits of a " + std::to_string(m) +
                       "x" + std::to_string(n) + " product need " + std::to_string(need) +
                       " bytes of partials, more than the library's " + std::to_string(have) + "-byte scratch";
        return 1;  // hipErrorInvalidValue
    }
    const int rc = mchip_launch_matmul_noalloc(kernel, a, b, c, m, n, k, stream, splits);
    if (rc != 0) g_last_error = std::string("mc_launch_matmul_noalloc: ") + mchip_error_string(rc);
    return rc;
}

MC_API unsigned long long mc_noalloc_scratch_bytes(void) { return mchip_noalloc_scratch_bytes(); }

MC_API int mc_launch_matmul_lowp(int kernel, int dtype, const void* a, const void* b, float* c, int m, int n, int k,
                                 void* stream, int splits, float* workspace) {
    return mchip_launch_matmul_lowp(kernel, dtype, a, b, c, m, n, k, stream, splits, workspace);
}

MC_API int mc_convert_f32(int dtype, const float* in, void* out, size_t count, void* stream) {
    return mchip_convert_f32(dtype, in, out, count, stream);
}

MC_API long long mc_packed_a16_bytes(int m, int k) { return 2 * mchip_packed_a16_elements(m, k); }

MC_API int mc_pack_a16(const void* a, void* packed, int m, int k, void* stream) {
    return mchip_pack_a16(a, packed, m, k, stream);
}

MC_API int mc_convert_pack_a_f32(int dtype, const float* a, void* packed, int m, int k, void* stream) {
    return mchip_convert_pack_a_f32(dtype, a, packed, m, k, stream);
}

MC_API int mc_launch_matmul_lowp_packed(int kernel, int dtype, const void* a_packed, const void* b, float* c, int m,
                                        int n, int k, void* stream) {
    return mchip_launch_matmul_lowp_packed(kernel, dtype, a_packed, b, c, m, n, k, stream);
}

MC_API int mc_sum_split_partials(const float* partial, float* c, size_t count, int splits, void* stream) {
    return mchip_sum_split_partials(partial, c, count, splits, stream);
}

MC_API int mc_split_k_splits(int m, int n, int k, int cu_count, int blocks_per_cu) {
    return hip::split_k_splits(m, n, k, cu_count, blocks_per_cu);
}

MC_API int mc_matmul_splits(int kernel, int m, int n, int k, int cu_count) {
    return hip::matmul_splits(static_cast<hip::MatmulKernel>(kernel), m, n, k, cu_count);
}

MC_API int mc_matmul_k_ranges(int kernel, int m, int n, int k, int splits) {
    return mchip_matmul_k_ranges(kernel, m, n, k, splits, MCHIP_RING_NONE);
}

MC_API long long mc_matmul_workspace_bytes(int kernel, int m, int n, int splits) {
    return static_cast<long long>(hip::matmul_workspace_bytes(static_cast<hip::MatmulKernel>(kernel), m, n, splits));
}

MC_API int mc_resolve_matmul_kernel(int kernel, int m, int n, int k, int cu_count) {
    return static_cast<int>(hip::resolve_matmul_kernel(static_cast<hip::MatmulKernel>(kernel), m, n, k, cu_count));
}

MC_API const char* mc_matmul_kernel_name(int kernel) {
    return hip::matmul_kernel_name(static_cast<hip::MatmulKernel>(kernel));
}

MC_API int mc_matmul_kernel_from_name(const char* name) {
    Result<hip::MatmulKernel> k = hip::matmul_kernel_from_name(name ? name : "");
    return k.ok() ? static_cast<int>(k.value()) : -1;
}

MC_API int mc_matmul_supported(int kernel) { return mchip_matmul_supported(kernel); }

MC_API int mc_device_count(void) {
    int n = 0;
    return mchip_device_count(&n) == 0 ? n : 0;
}
MC_API int mc_device_malloc(void** ptr, size_t bytes) { return mchip_malloc(ptr, bytes); }
MC_API int mc_device_free(void* ptr) { return mchip_free(ptr); }
MC_API int mc_memcpy_htod(void* dst, const void* src, size_t bytes) {
    const int rc = mchip_memcpy_htod_async(dst, src, bytes, nullptr);
    return rc ? rc : mchip_stream_synchronize(nullptr);
}
MC_API int mc_memcpy_dtoh(void* dst, const void* src, size_t bytes) { return mchip_memcpy_dtoh(dst, src, bytes); }
MC_API int mc_memcpy_dtod_async(void* dst, const void* src, size_t bytes, void* stream) {
    return mchip_memcpy_dtod_async(dst, src, bytes, stream);
}
MC_API int mc_memset(void* dst, int value, size_t bytes) {
    const int rc = mchip_memset_async(dst, value, bytes, nullptr);
    return rc ? rc : mchip_stream_synchronize(nullptr);
}
MC_API int mc_device_synchronize(void) { return mchip_device_synchronize(); }
MC_API int mc_stream_create(void** stream) { return mchip_stream_create(stream); }
MC_API int mc_stream_destroy(void* stream) { return mchip_stream_destroy(stream); }
MC_API int mc_stream_synchronize(void* stream) { return mchip_stream_synchronize(stream); }
MC_API int mc_event_create(void** event) { return mchip_event_create(event); }
MC_API int mc_event_destroy(void* event) { return mchip_event_destroy(event); }
MC_API int mc_event_record(void* event, void* stream) { return mchip_event_record(event, stream); }
MC_API int mc_event_elapsed_ms(void* start, void* stop, float* ms) { return mchip_event_elapsed_ms(ms, start, stop); }
MC_API int mc_stream_begin_capture(void* stream) { return mchip_capture_begin(stream); }
MC_API int mc_stream_end_capture(void* stream, void** graph_exec) { return mchip_capture_end(stream, graph_exec); }
MC_API int mc_graph_launch(void* graph_exec, void* stream) { return mchip_graph_launch(graph_exec, stream); }
MC_API int mc_graph_destroy(void* graph_exec) { return mchip_graph_exec_destroy(graph_exec); }

MC_API const char* mc_error_string(int code) { return mchip_error_string(code); }

}  // extern "C"
