// mcc: the minicompiler driver for this backend (the reference's
// tools/mcc.cpp:27-260 interface: parse a .mcg graph, run the passes, print,
// emit the generated kernels, run on seeded inputs, benchmark).

#include "hip/codegen.hpp"
#include "minicompiler/hip/hip_backend.hpp"
#include "minicompiler/parser.hpp"
#include "minicompiler/passes/pipeline.hpp"
#include "minicompiler/runtime/host_tensor.hpp"

#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <iostream>
#include <string>
#include <vector>

using namespace minicompiler;

namespace {

const char* kUsage = R"(usage: mcc GRAPH.mcg [options]

compile:
  --dim NAME=VALUE      override a dim declared in the graph (repeatable)
  --passes LIST         "default" (dne,fold,dne,fuse,dne), "none", or a list of dne, fold, fuse
  --print               print the optimized graph
  --emit-hip            print the HIP source generated for each elementwise node (no GPU needed)
  --stats               print node counts after each pass
  --matmul NAME         matmul kernel (auto, naive, tiled, register_tiled_128, register_tiled_64,
                        vectorized, double_buffered, split_k, tensor_core_bf16, tensor_core_f16)
  --no-vectorize        scalar elementwise accesses

run (backend hip):
  --run                 run once on seeded uniform(-1,1) inputs; print output checksums
  --seed N              input seed (default 1)
  --dump-outputs FILE   write the outputs as raw float32, concatenated
  --bench               time repeated enqueues (device-resident inputs); print JSON
  --warmup N            untimed runs before timing (default 10)
  --reps N              timed runs (default 50)

info:
  --list-backends       print the backends in this build
  --list-passes         print the available passes
)";

int die(const std::string& m) {
    std::cerr << "mcc: " << m << "\n";
    return 1;
}

std::string stats_line(const GraphStats& s) {
    return std::to_string(s.nodes) + " nodes, " + std::to_string(s.compute_nodes) + " compute (" +
           std::to_string(s.elementwise_ops) + " elementwise ops, " + std::to_string(s.matmuls) + " matmul, " +
           std::to_string(s.fused_nodes) + " fused kernels)";
}

}  // namespace

int main(int argc, char** argv) {
    std::vector<std::string> args(argv + 1, argv + argc);
    std::string path, passes = "default", dump;
    ParseOptions parse;
    hip::HipOptions hopt;
    bool print = false, emit = false, stats = false, run = false, bench = false;
    long long seed = 1, warmup = 10, reps = 50;
    for (std::size_t i = 0; i < args.size(); ++i) {
        const std::string& a = args[i];
        auto value = [&]() -> std::string {
            if (i + 1 >= args.size()) {
                std::cerr << "mcc: " << a << " needs a value\n";
                std::exit(1);
            }
            return args[++i];
        };
        if (a == "-h" || a == "--help") {
            std::cout << kUsage;
            return 0;
        } else if (a == "--list-backends") {
            for (const std::string& b : available_backends()) std::cout << b << "\n";
            return 0;
        } else if (a == "--list-passes") {
            for (const PassInfo& p : registered_passes()) std::cout << p.name << "\t" << p.description << "\n";
            return 0;
        } else if (a == "--dim") {
            const std::string d = value();
            const std::size_t eq = d.find('=');
            if (eq == std::string::npos) return die("bad --dim '" + d + "'");
            parse.dims[d.substr(0, eq)] = std::atoll(d.c_str() + eq + 1);
        } else if (a == "--passes") {
            passes = value();
        } else if (a == "--print") {
            print = true;
        } else if (a == "--emit-hip") {
            emit = true;
        } else if (a == "--stats") {
            stats = true;
        } else if (a == "--matmul") {
            Result<hip::MatmulKernel> k = hip::matmul_kernel_from_name(value());
            if (!k.ok()) return die(k.error().message);
            hopt.matmul = k.value();
        } else if (a == "--no-vectorize") {
            hopt.vectorize = false;
        } else if (a == "--backend") {
            const std::string b = value();
            if (b != "hip") return die("backend '" + b + "' is not in this build (available: hip)");
        } else if (a == "--run") {
            run = true;
        } else if (a == "--seed") {
            seed = std::atoll(value().c_str());
        } else if (a == "--dump-outputs") {
            dump = value();
            run = true;
        } else if (a == "--bench") {
            bench = true;
        } else if (a == "--warmup") {
            warmup = std::atoll(value().c_str());
        } else if (a == "--reps") {
            reps = std::atoll(value().c_str());
        } else if (!a.empty() && a[0] == '-') {
            return die("unknown option '" + a + "'");
        } else {
            path = a;
        }
    }
    if (path.empty()) return die("no graph file (see --help)");
    Result<Graph> g = parse_graph_file(path, parse);
    if (!g.ok()) return die(g.error().message);
    Result<std::vector<std::string>> pl = parse_pipeline(passes);
    if (!pl.ok()) return die(pl.error().message);
    std::vector<PassReport> reports;
    Result<Graph> opt = run_pipeline(g.value(), pl.value(), &reports);
    if (!opt.ok()) return die(opt.error().message);
    if (stats) {
        std::cout << "input: " << stats_line(compute_stats(g.value())) << "\n";
        for (const PassReport& r : reports) std::cout << r.pass << ": " << r.summary << "; " << stats_line(r.after) << "\n";
    }
    if (print) std::cout << print_graph(opt.value());
    if (emit) {
        for (const Node& n : opt->nodes()) {
            if (!is_elementwise(n.op) && n.op != OpKind::FusedElementwise) continue;
            const FusedProgram p = n.op == OpKind::FusedElementwise ? *n.fused : hip::single_op_program(n.op);
            std::vector<Shape> shapes;
            for (NodeId in : n.inputs) shapes.push_back(opt->node(in).type.shape);
            hip::CodegenOptions cg;
            cg.allow_vectorize = hopt.vectorize;
            std::cout << "// node " << n.name << "\n" << hip::generate_elementwise_kernel(p, shapes, n.type.shape, cg).source;
        }
    }
    if (!run && !bench) return 0;

    Result<std::unique_ptr<hip::HipExecutable>> exe = hip::compile_for_hip(opt.value(), hopt);
    if (!exe.ok()) return die(exe.error().message);
    const std::vector<HostTensor> inputs = make_random_inputs(opt.value(), static_cast<std::uint64_t>(seed));
    if (run) {
        std::vector<HostTensor> outputs;
        Status st = (*exe)->run(inputs, outputs);
        if (!st.ok()) return die(st.message());
        std::ofstream out;
        if (!dump.empty()) out.open(dump, std::ios::binary);
        for (std::size_t k = 0; k < outputs.size(); ++k) {
            double sum = 0, abs_sum = 0;
            for (float v : outputs[k].data) {
                sum += v;
                abs_sum += std::abs(v);
            }
            std::printf("output %zu %s: sum %.9g, sum|x| %.9g\n", k, to_string(outputs[k].type).c_str(), sum, abs_sum);
            if (out) out.write(reinterpret_cast<const char*>(outputs[k].data.data()),
                               static_cast<std::streamsize>(outputs[k].data.size() * sizeof(float)));
        }
    }
    if (bench) {
        std::vector<const float*> in;
        for (const HostTensor& t : inputs) in.push_back(t.data.data());
        Status st = (*exe)->upload_inputs(in);
        for (long long i = 0; st.ok() && i < warmup; ++i) st = (*exe)->enqueue();
        if (st.ok()) st = (*exe)->synchronize();
        std::vector<double> ms;
        for (long long i = 0; st.ok() && i < reps; ++i) {
            const auto t0 = std::chrono::steady_clock::now();
            st = (*exe)->enqueue();
            if (st.ok()) st = (*exe)->synchronize();
            ms.push_back(std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count());
        }
        if (!st.ok()) return die(st.message());
        std::sort(ms.begin(), ms.end());
        std::printf("{\"graph\":\"%s\",\"backend\":\"hip\",\"kernel_launches\":%zu,\"jit_compile_ms\":%.3f,"
                    "\"median_ms\":%.6f,\"min_ms\":%.6f,\"reps\":%lld}\n",
                    opt->name().c_str(), (*exe)->kernel_launches(), (*exe)->jit_compile_ms(),
                    ms.empty() ? 0.0 : ms[ms.size() / 2], ms.empty() ? 0.0 : ms.front(), reps);
    }
    return 0;
}
