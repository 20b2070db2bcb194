// The HIP executable and backend (replaces the reference's
// src/cuda/cuda_backend.cpp:52-366).
//
// Compile time (init): plan memory, lay every device allocation out in ONE
// arena (pooled plan buffers at their plan offsets, graph inputs, constants
// uploaded once, split-K workspaces; 256-byte aligned), generate and
// hipRTC-compile one kernel per elementwise node (concurrently), and build a
// flat launch list whose kernel arguments point at stable storage.
// Run time: enqueue() walks the list; no allocation, no host work beyond the
// launch calls. Inputs and outputs can be bound to caller device memory, in
// which case the kernels read and write it in place.

#include "minicompiler/hip/hip_backend.hpp"

#include "autotune.hpp"
#include "codegen.hpp"
#include "hip_rt.h"
#include "kernel_compiler.hpp"
#include "matmul.h"
#include "matmul_policy.hpp"
#include "rtc_sources.hpp"
#include "minicompiler/runtime/memory_plan.hpp"

#include <algorithm>
#include <atomic>
#include <cstdint>
#include <map>
#include <thread>

namespace minicompiler::hip {

namespace {

constexpr std::size_t kArenaAlign = 256;

std::size_t align_up(std::size_t v) { return (v + kArenaAlign - 1) / kArenaAlign * kArenaAlign; }

// Bytes of a converted tensor-core matmul's packed A (its workspace's first part).
template <class L>
std::size_t packed_a_bytes(const L& l) {
    return align_up(static_cast<std::size_t>(mchip_packed_a16_elements(l.m, l.k)) * 2);
}

Status hip_status(int rc, const char* call) {
    if (rc == 0) return Status();
    return Error{std::string(call) + ": " + mchip_error_string(rc)};
}

#define MCHIP_TRY(call)                                  \
    do {                                                 \
        const int mchip_rc_ = (call);                    \
        if (mchip_rc_ != 0) return hip_status(mchip_rc_, #call); \
    } while (0)

#define MCHIP_TRY_STATUS(expr)                \
    do {                                      \
        Status mchip_st_ = (expr);            \
        if (!mchip_st_.ok()) return mchip_st_; \
    } while (0)

bool is_tensor_core(MatmulKernel k) {
    return k == MatmulKernel::TensorCoreTf32 || k == MatmulKernel::TensorCoreBf16 || k == MatmulKernel::TensorCoreF16;
}

std::string arch_base(const std::string& arch) { return arch.substr(0, arch.find(':')); }

struct Launch {
    // FusedMatmul: an FP32 matrix-core GEMM whose store applies the fused
    // elementwise group `epilogue_node` (compiled at run time), writing that
    // group's output; with split K the epilogue runs in the split sum.
    enum class Kind { Elementwise, Matmul, FusedMatmul } kind = Kind::Elementwise;
    NodeId node = kNoNode;
    NodeId epilogue_node = kNoNode;
    // Elementwise: generated kernel, arguments out, in0.., count.
    void* function = nullptr;
    unsigned grid = 0;
    unsigned count = 0;
    std::vector<void*> ptrs;
    std::vector<void*> params;
    // Matmul.
    MatmulKernel matmul = MatmulKernel::DoubleBuffered;
    int splits = 1;
    int ring_cfg = 0;  // MCHIP_RING_*: forced FP32 ring configuration (0: the planner's)
    float* workspace = nullptr;
    // split_k: per-tile arrival counters (zeroed at init) when the GEMM
    // launch adds its splits' partials itself (split_fold), else null.
    unsigned* counters = nullptr;
    bool fold = false;  // FusedMatmul: the generated GEMM adds the partials (no sum launch)
    int m = 0, n = 0, k = 0;
    // FusedMatmul: generated kernels and their stable arguments.
    void* sum_function = nullptr;
    unsigned grid_x = 0, grid_y = 0, grid_z = 0, sum_grid = 0, block = 256;
    int k_split = 0, depth = 1;
    GemmBody body = GemmBody::F32Mfma;
    const void* a_ptr = nullptr;
    const void* b_ptr = nullptr;
    void* c_ptr = nullptr;
    void* partial = nullptr;
    std::vector<const void*> epilogue_inputs;  // the McEpilogue argument: one pointer per program input
    std::vector<void*> sum_params;
    // Tensor-core matmul on fp32 operands rounded to 16 bits in the launch's
    // workspace (a16, b16) first: per run, or once at compile time for a
    // constant operand. a16 holds A packed (mchip_convert_pack_a_f32: 256-row
    // bands of 16 KiB K-step blocks in the kernel's LDS order), b16 B row-major.
    bool lowp = false;
    int dtype = 0;
    void* a16 = nullptr;
    void* b16 = nullptr;
    bool convert_a = false, convert_b = false;
};

// K per split and number of splits as the FP32 matrix-core kernels lay them
// out (whole 32-wide K tiles per split).
void split_layout(int k, int splits, int* k_split, int* depth) {
    if (splits <= 1) {
        *k_split = std::max(k, 1);
    } else {
        const int per = (k + splits - 1) / splits;
        *k_split = (per + 31) / 32 * 32;
    }
    *depth = std::max(1, (k + *k_split - 1) / *k_split);
}

class HipExecutableImpl final : public HipExecutable {
    // graph_replay: per binding of caller memory, the captured enqueue and a
    // run of kGraphSteps captured enqueues.
    struct Captured {
        void* one = nullptr;
        void* run = nullptr;
    };
    static constexpr std::size_t kMaxCapturedBindings = 64;

public:
    HipExecutableImpl(const Graph& graph, const HipOptions& options)
        : graph_(graph), options_(options), plan_(plan_memory(graph_)) {}

    ~HipExecutableImpl() override {
        drop_graph();
        if (stream_) mchip_stream_destroy(stream_);
        if (arena_) mchip_free(arena_);
    }

    Status init() {
        Result<DeviceInfo> dev = query_device(options_.device);
        if (!dev.ok()) return dev.error();
        device_ = std::move(dev).value();
        MCHIP_TRY(mchip_set_device(options_.device));
        MCHIP_TRY(mchip_stream_create(&stream_));

        const std::size_t n = graph_.num_nodes();
        offset_.assign(n, 0);
        bound_.assign(n, nullptr);

        // Arena layout: plan buffers first, then inputs, constants, workspaces.
        std::vector<std::size_t> buffer_offset(plan_.buffer_bytes.size());
        std::size_t top = 0;
        for (std::size_t b = 0; b < plan_.buffer_bytes.size(); ++b) {
            buffer_offset[b] = top;
            top += align_up(std::max<std::size_t>(plan_.buffer_bytes[b], 4));
        }
        for (std::size_t i = 0; i < n; ++i) {
            const Node& node = graph_.node(static_cast<NodeId>(i));
            if (node.op == OpKind::Input || node.op == OpKind::Constant) {
                offset_[i] = top;
                top += align_up(std::max<std::size_t>(node.type.size_bytes(), 4));
            } else {
                offset_[i] = buffer_offset[static_cast<std::size_t>(plan_.buffer_of[i])];
            }
        }

        // Launches (matmul workspaces and split counters take arena space too).
        std::vector<std::size_t> workspace_offset, counter_offset;
        std::vector<bool> fused_away(n, false);
        for (std::size_t i = 0; i < n; ++i) {
            const auto id = static_cast<NodeId>(i);
            const Node& node = graph_.node(id);
            if (!is_compute(node.op) || fused_away[i]) continue;
            Launch l;
            l.node = id;
            if (node.op == OpKind::MatMul) {
                Status st = plan_matmul(node, &l);
                if (!st.ok()) return st;
                bool relocate = false;
                const NodeId f = epilogue_for(id, l, &relocate);
                if (f != kNoNode && relocate) {
                    // The group's planned buffer is one the fused kernel reads:
                    // its output gets arena space of its own instead.
                    offset_[static_cast<std::size_t>(f)] = top;
                    top += align_up(std::max<std::size_t>(graph_.node(f).type.size_bytes(), 4));
                }
                if (f != kNoNode) {
                    l.kind = Launch::Kind::FusedMatmul;
                    l.epilogue_node = f;
                    fused_away[static_cast<std::size_t>(f)] = true;
                    l.body = fused_body(l);
                }
                const std::size_t ws =
                    l.lowp ? packed_a_bytes(l) + align_up(static_cast<std::size_t>(l.k) * l.n * 2)
                           : matmul_workspace_bytes(l.matmul, l.m, l.n, l.splits);
                workspace_offset.push_back(ws ? top : SIZE_MAX);
                if (ws) top += align_up(ws);
                const std::size_t cb = ws && !l.lowp && options_.split_fold && l.matmul == MatmulKernel::SplitK
                                           ? static_cast<std::size_t>(mchip_split_counter_bytes(l.m, l.n))
                                           : 0;
                counter_offset.push_back(cb ? top : SIZE_MAX);
                if (cb) top += align_up(cb);
            } else {
                l.kind = Launch::Kind::Elementwise;
                workspace_offset.push_back(SIZE_MAX);
                counter_offset.push_back(SIZE_MAX);
            }
            launches_.push_back(std::move(l));
        }
        arena_bytes_ = std::max<std::size_t>(top, kArenaAlign);
        MCHIP_TRY(mchip_malloc(&arena_, arena_bytes_));
        auto* base = static_cast<char*>(arena_);
        for (std::size_t j = 0; j < launches_.size(); ++j) {
            if (workspace_offset[j] == SIZE_MAX) continue;
            Launch& l = launches_[j];
            if (l.lowp) {
                l.a16 = base + workspace_offset[j];
                l.b16 = base + workspace_offset[j] + packed_a_bytes(l);
            } else {
                l.workspace = reinterpret_cast<float*>(base + workspace_offset[j]);
            }
            if (counter_offset[j] != SIZE_MAX) {
                l.counters = reinterpret_cast<unsigned*>(base + counter_offset[j]);
                MCHIP_TRY(mchip_memset_async(l.counters, 0, static_cast<std::size_t>(mchip_split_counter_bytes(l.m, l.n)),
                                             stream_));
            }
        }
        // Constants are uploaded once, here.
        for (std::size_t i = 0; i < n; ++i) {
            const Node& node = graph_.node(static_cast<NodeId>(i));
            if (node.op != OpKind::Constant) continue;
            MCHIP_TRY(mchip_memcpy_htod_async(base + offset_[i], node.constant->data(), node.type.size_bytes(), stream_));
        }
        // Constant operands of converted tensor-core matmuls: rounded once, here.
        for (const Launch& l : launches_) {
            if (!l.lowp) continue;
            if (!l.convert_a) {
                MCHIP_TRY(mchip_convert_pack_a_f32(l.dtype, static_cast<const float*>(value_ptr(a_of(l))), l.a16, l.m,
                                                   l.k, stream_));
            }
            if (!l.convert_b) {
                MCHIP_TRY(mchip_convert_f32(l.dtype, static_cast<const float*>(value_ptr(b_of(l))), l.b16,
                                            static_cast<std::size_t>(l.k) * l.n, stream_));
            }
        }
        MCHIP_TRY(mchip_stream_synchronize(stream_));

        Status st = build_elementwise();
        if (!st.ok()) return st;
        refresh_pointers();
        return Status();
    }

    // Executable

    Status run(const std::vector<HostTensor>& inputs, std::vector<HostTensor>& outputs) override {
        if (&inputs == &outputs) return Error{"run() needs separate input and output vectors"};
        if (inputs.size() != graph_.inputs().size()) {
            return Error{"expected " + std::to_string(graph_.inputs().size()) + " inputs, got " +
                         std::to_string(inputs.size())};
        }
        std::vector<const float*> in;
        for (std::size_t k = 0; k < inputs.size(); ++k) {
            const Node& node = graph_.node(graph_.inputs()[k]);
            if (inputs[k].type != node.type || inputs[k].data.size() != node.type.num_elements()) {
                return Error{"input '" + node.name + "' should be " + to_string(node.type) + ", got " +
                             to_string(inputs[k].type)};
            }
            in.push_back(inputs[k].data.data());
        }
        outputs.resize(graph_.outputs().size());
        std::vector<float*> out;
        for (std::size_t k = 0; k < outputs.size(); ++k) {
            const TensorType& t = graph_.node(graph_.outputs()[k]).type;
            outputs[k].type = t;
            outputs[k].data.resize(t.num_elements());
            out.push_back(outputs[k].data.data());
        }
        return run_buffers(in, out);
    }

    Status run_buffers(const std::vector<const float*>& inputs, const std::vector<float*>& outputs) override {
        if (inputs.size() != graph_.inputs().size() || outputs.size() != graph_.outputs().size()) {
            return Error{"expected " + std::to_string(graph_.inputs().size()) + " input and " +
                         std::to_string(graph_.outputs().size()) + " output buffers"};
        }
        Status st = upload_inputs(inputs);
        if (st.ok()) st = enqueue(nullptr);
        if (st.ok()) st = download_outputs(outputs);
        return st;
    }

    std::size_t intermediate_bytes() const override { return plan_.bytes_with_reuse(); }

    // HipExecutable

    Status upload_inputs(const std::vector<const float*>& host_inputs) override {
        if (host_inputs.size() != graph_.inputs().size()) return Error{"wrong number of inputs"};
        MCHIP_TRY(mchip_set_device(options_.device));
        for (std::size_t k = 0; k < host_inputs.size(); ++k) {
            const NodeId id = graph_.inputs()[k];
            MCHIP_TRY(mchip_memcpy_htod_async(value_ptr(id), host_inputs[k], graph_.node(id).type.size_bytes(), stream_));
        }
        // Kernels may be enqueued on another stream, which would not wait.
        MCHIP_TRY(mchip_stream_synchronize(stream_));
        return Status();
    }

    Status enqueue(void* stream) override {
        if (!options_.graph_replay) return enqueue_with_events(stream, nullptr);
        void* s = stream ? stream : stream_;
        Captured& cap = captured_for_binding();
        if (cap.one == nullptr) MCHIP_TRY_STATUS(capture_steps(s, 1, &cap.one));
        MCHIP_TRY(mchip_graph_launch(cap.one, s));
        graphs_launched_ = true;
        return Status();
    }

    Status enqueue_steps(int count, void* stream) override {
        if (count < 0) return Error{"enqueue_steps: negative count"};
        void* s = stream ? stream : stream_;
        int done = 0;
        if (options_.graph_replay && count >= kGraphSteps) {
            // One hipGraphLaunch costs more host time than the two or three
            // launches of a small graph's step (19-26 us on an MI355X against
            // 5.3 us), so single-step replays leave the GPU waiting; a run of
            // kGraphSteps steps pays it once.
            Captured& cap = captured_for_binding();
            if (cap.run == nullptr) MCHIP_TRY_STATUS(capture_steps(s, kGraphSteps, &cap.run));
            for (; done + kGraphSteps <= count; done += kGraphSteps) MCHIP_TRY(mchip_graph_launch(cap.run, s));
            graphs_launched_ = true;
        }
        for (; done < count; ++done) MCHIP_TRY_STATUS(enqueue(s));
        return Status();
    }

    // Captures `steps` consecutive enqueues on `s` into an executable graph.
    Status capture_steps(void* s, int steps, void** out) {
        MCHIP_TRY(mchip_capture_begin(s));
        Status st;
        for (int i = 0; i < steps && st.ok(); ++i) st = enqueue_with_events(s, nullptr);
        void* exec = nullptr;
        const int rc = mchip_capture_end(s, &exec);  // ends the capture also after a failed launch
        if (!st.ok()) {
            if (exec) mchip_graph_exec_destroy(exec);
            return st;
        }
        if (rc != 0) return hip_status(rc, "hipStreamEndCapture / hipGraphInstantiate");
        *out = exec;
        return Status();
    }

    Status enqueue_with_events(void* stream, void* const* events) override {
        void* s = stream ? stream : stream_;
        std::size_t j = 0;
        for (Launch& l : launches_) {
            if (events) MCHIP_TRY(mchip_event_record(events[j++], s));
            Status st = launch(l, s);
            if (!st.ok()) return st;
        }
        if (events) MCHIP_TRY(mchip_event_record(events[j], s));
        // Graph outputs that are inputs or constants: copy into bound memory.
        for (std::size_t k = 0; k < graph_.outputs().size(); ++k) {
            const NodeId id = graph_.outputs()[k];
            if (is_compute(graph_.node(id).op) || output_bound_[k] == nullptr) continue;
            MCHIP_TRY(mchip_memcpy_dtod_async(output_bound_[k], value_ptr(id), graph_.node(id).type.size_bytes(), s));
        }
        return Status();
    }

    Status enqueue_launch(std::size_t j, void* stream) override {
        if (j >= launches_.size()) return Error{"launch " + std::to_string(j) + " out of range"};
        return launch(launches_[j], stream ? stream : stream_);
    }

    Status synchronize() override {
        MCHIP_TRY(mchip_set_device(options_.device));
        MCHIP_TRY(mchip_device_synchronize());
        return Status();
    }

    Status download_outputs(const std::vector<float*>& host_outputs) override {
        if (host_outputs.size() != graph_.outputs().size()) return Error{"wrong number of outputs"};
        MCHIP_TRY(mchip_set_device(options_.device));
        // Kernels may have gone to a caller's stream: wait for the device.
        MCHIP_TRY(mchip_device_synchronize());
        for (std::size_t k = 0; k < host_outputs.size(); ++k) {
            const NodeId id = graph_.outputs()[k];
            const void* src = output_bound_[k] ? output_bound_[k] : value_ptr(id);
            MCHIP_TRY(mchip_memcpy_dtoh(host_outputs[k], src, graph_.node(id).type.size_bytes()));
        }
        return Status();
    }

    Status bind_inputs(const std::vector<const void*>& device_inputs) override {
        if (device_inputs.size() != graph_.inputs().size()) return Error{"wrong number of inputs to bind"};
        for (const void* p : device_inputs) {
            if (reinterpret_cast<std::uintptr_t>(p) % 16 != 0) return Error{"bound inputs must be 16-byte aligned"};
        }
        for (std::size_t k = 0; k < device_inputs.size(); ++k) {
            bound_[static_cast<std::size_t>(graph_.inputs()[k])] = const_cast<void*>(device_inputs[k]);
        }
        refresh_pointers();
        return Status();
    }

    Status bind_outputs(const std::vector<void*>& device_outputs) override {
        if (device_outputs.size() != graph_.outputs().size()) return Error{"wrong number of outputs to bind"};
        for (void* p : device_outputs) {
            if (reinterpret_cast<std::uintptr_t>(p) % 16 != 0) return Error{"bound outputs must be 16-byte aligned"};
        }
        for (std::size_t k = 0; k < device_outputs.size(); ++k) {
            const NodeId id = graph_.outputs()[k];
            output_bound_[k] = device_outputs[k];
            if (is_compute(graph_.node(id).op)) bound_[static_cast<std::size_t>(id)] = device_outputs[k];
        }
        refresh_pointers();
        return Status();
    }

    void* input_device_ptr(std::size_t k) const override {
        return k < graph_.inputs().size() ? value_ptr(graph_.inputs()[k]) : nullptr;
    }
    void* output_device_ptr(std::size_t k) const override {
        if (k >= graph_.outputs().size()) return nullptr;
        return output_bound_[k] ? output_bound_[k] : value_ptr(graph_.outputs()[k]);
    }

    void* stream() const override { return stream_; }

    std::size_t kernel_launches() const override { return launches_.size(); }
    std::vector<std::string> kernel_sources() const override { return sources_; }
    std::vector<std::string> launch_names() const override {
        std::vector<std::string> names;
        for (const Launch& l : launches_) {
            const Node& node = graph_.node(l.node);
            if (l.kind == Launch::Kind::Matmul || l.kind == Launch::Kind::FusedMatmul) {
                // The K ranges that run (the split count is an upper bound
                // for the narrow-tile body), and the count asked for when
                // they differ.
                const int ranges = l.kind == Launch::Kind::FusedMatmul || l.lowp
                                       ? (l.lowp ? 1 : l.depth)
                                       : mchip_matmul_k_ranges(static_cast<int>(l.matmul), l.m, l.n, l.k, l.splits,
                                                               l.ring_cfg);
                std::string name = std::string("matmul ") + matmul_kernel_name(l.matmul) + " " + std::to_string(l.m) +
                                   "x" + std::to_string(l.n) + "x" + std::to_string(l.k);
                if (l.splits > 1 || ranges > 1) {
                    name += " splits=" + std::to_string(ranges);
                    if (ranges != l.splits) name += " of " + std::to_string(l.splits);
                }
                if (folds(l)) name += ", summed in the GEMM";
                if (l.kind == Launch::Kind::FusedMatmul) {
                    const Node& f = graph_.node(l.epilogue_node);
                    name += " + fused " + f.name + " " + to_string(f.type);
                }
                names.push_back(name);
            } else {
                names.push_back(std::string(op_name(node.op)) + " " + node.name + " " + to_string(node.type));
            }
        }
        return names;
    }
    std::vector<std::vector<NodeId>> launch_nodes() const override {
        std::vector<std::vector<NodeId>> out;
        for (const Launch& l : launches_) {
            out.push_back({l.node});
            if (l.kind == Launch::Kind::FusedMatmul) out.back().push_back(l.epilogue_node);
        }
        return out;
    }
    std::vector<MatmulKernel> matmul_kernels() const override {
        std::vector<MatmulKernel> ks;
        for (const Launch& l : launches_) {
            if (l.kind == Launch::Kind::Matmul || l.kind == Launch::Kind::FusedMatmul) ks.push_back(l.matmul);
        }
        return ks;
    }
    double jit_compile_ms() const override { return jit_ms_; }
    std::size_t arena_bytes() const override { return arena_bytes_; }

private:
    Status launch(Launch& l, void* s) {
        if (l.kind == Launch::Kind::Elementwise) {
            const int rc = mchip_module_launch(l.function, l.grid, kElementwiseBlock, 0, s, l.params.data());
            return rc == 0 ? Status() : hip_status(rc, "hipModuleLaunchKernel");
        }
        if (l.lowp) {
            int rc = 0;
            if (l.convert_a) {
                rc = mchip_convert_pack_a_f32(l.dtype, static_cast<const float*>(value_ptr(a_of(l))), l.a16, l.m, l.k,
                                              s);
            }
            if (rc == 0 && l.convert_b) {
                rc = mchip_convert_f32(l.dtype, static_cast<const float*>(value_ptr(b_of(l))), l.b16,
                                       static_cast<std::size_t>(l.k) * l.n, s);
            }
            if (rc != 0) return hip_status(rc, "convert_f32");
            if (l.kind == Launch::Kind::FusedMatmul) {
                rc = mchip_module_launch(l.function, l.grid_x, 512, 0, s, l.params.data());
                return rc == 0 ? Status() : hip_status(rc, "hipModuleLaunchKernel(mc_gemm_epilogue)");
            }
            rc = mchip_launch_matmul_lowp_packed(static_cast<int>(l.matmul), l.dtype, l.a16, l.b16,
                                                 static_cast<float*>(value_ptr(l.node)), l.m, l.n, l.k, s);
            if (rc != 0) {
                return Error{std::string("launch_matmul_lowp_packed(") + matmul_kernel_name(l.matmul) + "): " +
                             mchip_error_string(rc)};
            }
            return Status();
        }
        if (l.kind == Launch::Kind::FusedMatmul) {
            int rc = mchip_module_launch3(l.function, l.grid_x, l.grid_y, l.grid_z, l.block, 0, s, l.params.data());
            if (rc != 0) return hip_status(rc, "hipModuleLaunchKernel(mc_gemm_epilogue)");
            if (l.depth > 1 && !l.fold) {
                rc = mchip_module_launch(l.sum_function, l.sum_grid, 256, 0, s, l.sum_params.data());
                if (rc != 0) return hip_status(rc, "hipModuleLaunchKernel(mc_sum_splits_epilogue)");
            }
            return Status();
        }
        const void* pa = value_ptr(a_of(l));
        const void* pb = value_ptr(b_of(l));
        void* pc = value_ptr(l.node);
        // A tuned ring configuration needs 16-byte aligned operands (bound
        // caller buffers may not be); the planner's own choice runs any.
        const bool aligned = ((reinterpret_cast<std::uintptr_t>(pa) | reinterpret_cast<std::uintptr_t>(pb) |
                               reinterpret_cast<std::uintptr_t>(pc)) & 15u) == 0;
        const int rc = mchip_launch_matmul_fold(static_cast<int>(l.matmul), static_cast<const float*>(pa),
                                                static_cast<const float*>(pb), static_cast<float*>(pc), l.m, l.n, l.k,
                                                s, l.splits, l.workspace, aligned ? l.ring_cfg : 0, l.counters);
        if (rc != 0) {
            return Error{std::string("launch_matmul(") + matmul_kernel_name(l.matmul) + "): " + mchip_error_string(rc)};
        }
        return Status();
    }

    // Whether the launch adds its K splits' partials itself (no sum launch),
    // for 16-byte aligned operands (arena buffers always are).
    bool folds(const Launch& l) const {
        if (l.kind == Launch::Kind::FusedMatmul) return l.fold;
        return l.kind == Launch::Kind::Matmul && l.counters != nullptr &&
               mchip_split_k_folds(l.m, l.n, l.k, l.splits, l.ring_cfg) != 0;
    }

    // graph_replay: a captured graph holds the kernel arguments of the time
    // of capture, so graphs are kept per binding of caller memory (bound
    // inputs and outputs): a caller cycling through buffer sets replays one
    // graph per set, and a rebinding never destroys a graph that may run.
    std::vector<void*> binding_key() const {
        std::vector<void*> key(bound_);
        key.insert(key.end(), output_bound_.begin(), output_bound_.end());
        return key;
    }
    Captured& captured_for_binding() {
        std::vector<void*> key = binding_key();
        auto it = captured_.find(key);
        if (it == captured_.end()) {
            if (captured_.size() >= kMaxCapturedBindings) drop_graph();
            it = captured_.emplace(std::move(key), Captured{}).first;
        }
        return it->second;
    }

    // Destroys every captured graph, after the device has finished whatever
    // of them was launched (a graph may be in flight on any stream).
    void drop_graph() {
        if (graphs_launched_) (void)mchip_device_synchronize();
        graphs_launched_ = false;
        for (auto& kv : captured_) {
            if (kv.second.one) mchip_graph_exec_destroy(kv.second.one);
            if (kv.second.run) mchip_graph_exec_destroy(kv.second.run);
        }
        captured_.clear();
    }

    NodeId a_of(const Launch& l) const { return graph_.node(l.node).inputs[0]; }
    NodeId b_of(const Launch& l) const { return graph_.node(l.node).inputs[1]; }

    void* value_ptr(NodeId id) const {
        const auto i = static_cast<std::size_t>(id);
        if (bound_[i]) return bound_[i];
        return static_cast<char*>(arena_) + offset_[i];
    }

    Status plan_matmul(const Node& node, Launch* l) {
        const Shape& a = graph_.node(node.inputs[0]).type.shape;
        l->kind = Launch::Kind::Matmul;
        l->m = static_cast<int>(a[0]);
        l->k = static_cast<int>(a[1]);
        l->n = static_cast<int>(node.type.shape[1]);
        l->matmul = resolve_matmul_kernel(options_.matmul, l->m, l->n, l->k, device_.cu_count);
        if (is_tensor_core(l->matmul) && !mchip_matmul_supported(static_cast<int>(l->matmul))) {
            return Error{std::string("matmul kernel '") + matmul_kernel_name(l->matmul) + "' does not run on " +
                         device_.name + " (" + device_.arch +
                         "): gfx950 has bf16 and fp16 matrix instructions but no xf32 (TF32) one"};
        }
        l->splits = uses_split_k(l->matmul) ? matmul_splits(l->matmul, l->m, l->n, l->k, device_.cu_count) : 1;
        if (options_.ring_config == MCHIP_RING_NARROW) {
            // The narrow-tile body: split_k only, K a multiple of 16.
            if (l->matmul == MatmulKernel::SplitK && l->k % 16 == 0 && l->n % 4 == 0) l->ring_cfg = MCHIP_RING_NARROW;
        } else if ((l->matmul == MatmulKernel::DoubleBuffered || l->matmul == MatmulKernel::SplitK) &&
                   l->k % 32 == 0 && l->n % 4 == 0) {
            l->ring_cfg = options_.ring_config;  // a shape the ring cannot take keeps the planner's body
        }
        if (options_.autotune && options_.matmul == MatmulKernel::Auto) {
            // The split count and ring configuration timed on this device
            // (double_buffered unsplit, split_k otherwise) instead of the
            // split rule's count and the planner's configuration.
            Result<Fp32Choice> tuned = autotune_fp32(device_, l->m, l->n, l->k, options_.split_fold);
            if (!tuned.ok()) return tuned.error();
            l->splits = tuned->splits;
            l->ring_cfg = tuned->ring_cfg;
            l->matmul = l->splits > 1 ? MatmulKernel::SplitK : MatmulKernel::DoubleBuffered;
        }
        const bool bf16 = l->matmul == MatmulKernel::TensorCoreBf16, f16 = l->matmul == MatmulKernel::TensorCoreF16;
        if (options_.convert_tensor_core_operands && (bf16 || f16) && mchip_mfma16_fast_fits(l->m, l->n, l->k)) {
            l->lowp = true;
            l->splits = 1;
            l->dtype = bf16 ? MCHIP_DTYPE_BF16 : MCHIP_DTYPE_F16;
            l->convert_a = graph_.node(node.inputs[0]).op != OpKind::Constant;
            l->convert_b = graph_.node(node.inputs[1]).op != OpKind::Constant;
        }
        return Status();
    }

    // The GEMM body of a fused matmul, chosen as mchip_launch_matmul chooses
    // for the same kernel (operands in the arena or bound by the caller are
    // 16-byte aligned).
    GemmBody fused_body(Launch& l) const {
        if (l.lowp) return l.dtype == MCHIP_DTYPE_BF16 ? GemmBody::Bf16Fast : GemmBody::F16Fast;
        if (l.matmul == MatmulKernel::SplitK &&
            (l.ring_cfg == MCHIP_RING_NONE || l.ring_cfg == MCHIP_RING_NARROW)) {
            int shape = 0, splits = 0, k_split = 0;
            if (mchip_f32_narrow_plan(l.m, l.n, l.k, std::max(l.splits, 1), device_.cu_count,
                                      l.ring_cfg == MCHIP_RING_NARROW, &shape, &splits, &k_split)) {
                l.k_split = k_split;
                l.depth = splits;
                switch (shape) {
                    case MCHIP_NARROW_16X64_STREAM: return GemmBody::F32Narrow16;
                    case MCHIP_NARROW_16X64: return GemmBody::F32Narrow16x64;
                    case MCHIP_NARROW_16X32: return GemmBody::F32Narrow16x32;
                    case MCHIP_NARROW_64X64: return GemmBody::F32Narrow64;
                    default: return GemmBody::F32Narrow32;
                }
            }
        }
        split_layout(l.k, l.splits, &l.k_split, &l.depth);
        if (l.matmul == MatmulKernel::Vectorized || l.k % 4 != 0) return GemmBody::F32Mfma;
        unsigned grid = 0, block = 0;
        switch (mchip_f32_ring_plan_cfg(l.m, l.n, l.k, l.depth, device_.cu_count, l.ring_cfg, &grid, &block)) {
            case MCHIP_RING_BIG: return GemmBody::F32RingBig;
            case MCHIP_RING_THIN: return GemmBody::F32RingThin;
            case MCHIP_RING_WIDE: return GemmBody::F32RingWide;
            case MCHIP_RING_WIDE8:
                if (l.ring_cfg == MCHIP_RING_WIDE8) return GemmBody::F32RingWide8;
                // The planner's 8-wave choice, with a group in the store: the
                // 4-wave blocks are faster there (the MLP's GEMM2 with b2 +
                // residual, 140.9 against 142.9 us on an MI355X).
                l.ring_cfg = MCHIP_RING_WIDE;
                return GemmBody::F32RingWide;
            case MCHIP_RING_MID: return GemmBody::F32RingMid;
            default: return GemmBody::F32Mfma;
        }
    }

    // The fused elementwise group this matmul's store can apply, or kNoNode.
    // Only when it is safe to run the group at the matmul's place: the group
    // is the next compute node, reads the product element for element (same
    // element count) and is its only reader, and the product is not a graph
    // output. The memory plan may hand a buffer freed by the matmul's
    // operands (or by another input of the group) to the group's output; then
    // *relocate is set and the output must be placed outside the plan's
    // buffers, since the fused kernel still reads that buffer.
    NodeId epilogue_for(NodeId m, const Launch& l, bool* relocate) const {
        *relocate = false;
        if (!options_.fuse_epilogue) return kNoNode;
        if (!l.lowp && l.matmul != MatmulKernel::Vectorized && l.matmul != MatmulKernel::DoubleBuffered &&
            l.matmul != MatmulKernel::SplitK) {
            return kNoNode;
        }
        for (NodeId o : graph_.outputs()) {
            if (o == m) return kNoNode;
        }
        NodeId f = kNoNode;
        for (std::size_t j = static_cast<std::size_t>(m) + 1; j < graph_.num_nodes(); ++j) {
            if (is_compute(graph_.node(static_cast<NodeId>(j)).op)) {
                f = static_cast<NodeId>(j);
                break;
            }
        }
        if (f == kNoNode) return kNoNode;
        const Node& fn = graph_.node(f);
        if (fn.op != OpKind::FusedElementwise || fn.type.num_elements() != graph_.node(m).type.num_elements()) {
            return kNoNode;
        }
        std::size_t readers = 0;
        for (std::size_t j = 0; j < graph_.num_nodes(); ++j) {
            for (NodeId in : graph_.node(static_cast<NodeId>(j)).inputs) readers += in == m ? 1 : 0;
        }
        if (readers != 1) return kNoNode;
        const std::int32_t out_buffer = plan_.buffer_of[static_cast<std::size_t>(f)];
        auto shares_output_buffer = [&](NodeId id) {
            const Node& node = graph_.node(id);
            if (node.op == OpKind::Input || node.op == OpKind::Constant) return false;
            return plan_.buffer_of[static_cast<std::size_t>(id)] == out_buffer;
        };
        for (NodeId in : graph_.node(m).inputs) *relocate = *relocate || shares_output_buffer(in);
        for (NodeId in : fn.inputs) *relocate = *relocate || (in != m && shares_output_buffer(in));
        return f;
    }

    // Generates every elementwise kernel and compiles them concurrently.
    Status build_elementwise() {
        struct Job {
            std::size_t launch;
            ElementwiseKernel kernel;
        };
        std::vector<Job> jobs;
        const CodegenOptions cg = codegen_options(options_);
        for (std::size_t j = 0; j < launches_.size(); ++j) {
            if (launches_[j].kind == Launch::Kind::FusedMatmul) {
                const Launch& l = launches_[j];
                const Node& f = graph_.node(l.epilogue_node);
                std::vector<Shape> shapes;
                std::size_t acc = 0;
                for (std::size_t k = 0; k < f.inputs.size(); ++k) {
                    shapes.push_back(graph_.node(f.inputs[k]).type.shape);
                    if (f.inputs[k] == l.node) acc = k;
                }
                ElementwiseKernel k;
                const GemmBody body = l.body;
                const char* body_source = l.lowp                        ? kGemm16FastSource
                                          : body == GemmBody::F32Mfma ? kGemmF32MfmaSource
                                          : is_narrow_body(body)      ? kGemmF32NarrowSource
                                                                      : kGemmF32RingSource;
                GemmDims dims;
                dims.m = l.m;
                dims.n = l.n;
                dims.k = l.k;
                dims.k_split = l.k_split;
                dims.depth = l.depth;
                k.source = generate_gemm_epilogue_kernel(*f.fused, acc, shapes, f.type.shape, l.n % 4 == 0 && l.k % 4 == 0,
                                                         body_source, body, dims)
                               .source;
                jobs.push_back({j, std::move(k)});
                continue;
            }
            if (launches_[j].kind != Launch::Kind::Elementwise) continue;
            const Node& node = graph_.node(launches_[j].node);
            const FusedProgram program =
                node.op == OpKind::FusedElementwise ? *node.fused : single_op_program(node.op);
            std::vector<Shape> shapes;
            for (NodeId in : node.inputs) shapes.push_back(graph_.node(in).type.shape);
            jobs.push_back({j, generate_elementwise_kernel(program, shapes, node.type.shape, cg)});
        }
        const std::string arch = arch_base(device_.arch);
        const int dev = options_.device;
        std::vector<Result<CompiledKernel>> built(jobs.size(), Result<CompiledKernel>(Error{"not compiled"}));
        std::vector<double> ms(jobs.size(), 0.0);
        const std::size_t workers =
            std::max<std::size_t>(1, std::min<std::size_t>(jobs.size(), std::min(16u, std::max(1u, std::thread::hardware_concurrency()))));
        std::vector<std::thread> pool;
        std::atomic<std::size_t> next{0};
        for (std::size_t w = 0; w < workers; ++w) {
            pool.emplace_back([&]() {
                mchip_set_device(dev);  // per thread
                for (std::size_t j = next++; j < jobs.size(); j = next++) {
                    const bool gemm = launches_[jobs[j].launch].kind == Launch::Kind::FusedMatmul;
                    built[j] = KernelCompiler::instance().get(jobs[j].kernel.source,
                                                              gemm ? kGemmEpilogueKernelName : kElementwiseKernelName,
                                                              arch, dev, &ms[j]);
                }
            });
        }
        for (std::thread& t : pool) t.join();
        for (std::size_t j = 0; j < jobs.size(); ++j) {
            if (!built[j].ok()) return built[j].error();
            Launch& l = launches_[jobs[j].launch];
            const ElementwiseKernel& kern = jobs[j].kernel;
            jit_ms_ += ms[j];
            sources_.push_back(kern.source);
            if (l.kind == Launch::Kind::FusedMatmul && l.lowp) {
                l.function = built[j]->function;
                l.grid_x = mchip_mfma16_fast_grid(l.m, l.n, device_.cu_count);
                l.grid_y = l.grid_z = 1;
                l.epilogue_inputs.assign(graph_.node(l.epilogue_node).inputs.size(), nullptr);
                continue;
            }
            if (l.kind == Launch::Kind::FusedMatmul) {
                l.function = built[j]->function;
                Result<CompiledKernel> sum = KernelCompiler::instance().get(kern.source, kSumSplitsEpilogueKernelName,
                                                                            arch, dev, nullptr);
                if (!sum.ok()) return sum.error();
                l.sum_function = sum->function;
                if (l.body == GemmBody::F32Mfma) {
                    l.grid_x = static_cast<unsigned>((l.n + 127) / 128);
                    l.grid_y = static_cast<unsigned>((l.m + 127) / 128);
                    l.grid_z = static_cast<unsigned>(l.depth);
                    l.block = 256;
                } else if (is_narrow_body(l.body)) {
                    // One-dimensional: the body maps blocks to tiles XCD by XCD.
                    const int rows = narrow_rows(l.body), cols = narrow_cols(l.body);
                    l.grid_x = static_cast<unsigned>(((l.n + cols - 1) / cols) * l.depth * ((l.m + rows - 1) / rows));
                    l.grid_y = l.grid_z = 1;
                    l.block = 256;
                } else {
                    unsigned grid = 0, block = 0;
                    mchip_f32_ring_plan_cfg(l.m, l.n, l.k, l.depth, device_.cu_count, l.ring_cfg, &grid, &block);
                    l.grid_x = grid;
                    l.grid_y = l.grid_z = 1;
                    l.block = block;
                }
                l.count = static_cast<unsigned>(static_cast<std::size_t>(l.m) * l.n);
                l.sum_grid = static_cast<unsigned>(std::max<std::size_t>(
                    1, std::min<std::size_t>((static_cast<std::size_t>(l.count) + 255) / 256, 8192)));
                l.partial = l.depth > 1 ? l.workspace : nullptr;
                l.fold = l.depth > 1 && l.counters != nullptr && l.body != GemmBody::F32Mfma;
                if (!l.fold) l.counters = nullptr;
                l.epilogue_inputs.assign(graph_.node(l.epilogue_node).inputs.size(), nullptr);
                continue;
            }
            const std::size_t numel = graph_.node(l.node).type.num_elements();
            l.function = built[j]->function;
            l.count = static_cast<unsigned>(kern.vectorized ? numel / 4 : numel);
            // Blocks per CU of the grid (those past what fits at once run in
            // turn), capped by the work: by default enough for one loop step
            // per block up to 64 per CU. A block that stores and exits lets a
            // fresh one issue its loads at once, where a looping wave's next
            // loads wait behind its stores (one counter holds both); on an
            // MI355X BatchNorm [200704,256] ran at 6.2 TB/s against 6.0 with
            // the resident grid (8 per CU), GELU and copy the same.
            int per_cu = static_cast<int>(options_.elementwise_blocks_per_cu);
            if (per_cu == 0) per_cu = kElementwiseBlocksPerCu;
            const std::size_t per_step = kern.items_per_block_step();
            const std::size_t needed = (static_cast<std::size_t>(l.count) + per_step - 1) / per_step;
            const std::size_t resident = std::max<std::size_t>(1, static_cast<std::size_t>(per_cu) * device_.cu_count);
            l.grid = static_cast<unsigned>(std::max<std::size_t>(1, std::min(needed, resident)));
            l.ptrs.assign(1 + graph_.node(l.node).inputs.size(), nullptr);
        }
        // Stable argument addresses: the launch list no longer changes.
        for (Launch& l : launches_) {
            if (l.kind == Launch::Kind::FusedMatmul && l.lowp) {
                l.params = {&l.a16, &l.b16, &l.c_ptr, &l.m, &l.n, &l.k, l.epilogue_inputs.data()};
                continue;
            }
            if (l.kind == Launch::Kind::FusedMatmul) {
                l.params = {&l.a_ptr, &l.b_ptr, &l.c_ptr, &l.m, &l.n, &l.k, &l.k_split, &l.depth, &l.partial,
                            &l.counters, l.epilogue_inputs.data()};
                l.sum_params = {&l.partial, &l.c_ptr, &l.count, &l.depth, l.epilogue_inputs.data()};
                continue;
            }
            if (l.kind != Launch::Kind::Elementwise) continue;
            for (void*& p : l.ptrs) l.params.push_back(&p);
            l.params.push_back(&l.count);
        }
        return Status();
    }

    void refresh_pointers() {
        if (output_bound_.size() != graph_.outputs().size()) output_bound_.assign(graph_.outputs().size(), nullptr);
        for (Launch& l : launches_) {
            if (l.kind == Launch::Kind::FusedMatmul) {
                l.a_ptr = value_ptr(a_of(l));
                l.b_ptr = value_ptr(b_of(l));
                l.c_ptr = value_ptr(l.epilogue_node);
                const Node& f = graph_.node(l.epilogue_node);
                for (std::size_t k = 0; k < f.inputs.size(); ++k) {
                    l.epilogue_inputs[k] = f.inputs[k] == l.node ? nullptr : value_ptr(f.inputs[k]);
                }
                continue;
            }
            if (l.kind != Launch::Kind::Elementwise) continue;
            const Node& node = graph_.node(l.node);
            l.ptrs[0] = value_ptr(l.node);
            for (std::size_t k = 0; k < node.inputs.size(); ++k) l.ptrs[k + 1] = value_ptr(node.inputs[k]);
        }
    }

    Graph graph_;
    HipOptions options_;
    MemoryPlan plan_;
    DeviceInfo device_;
    void* stream_ = nullptr;
    std::map<std::vector<void*>, Captured> captured_;
    bool graphs_launched_ = false;  // since the last drop_graph
    void* arena_ = nullptr;
    std::size_t arena_bytes_ = 0;
    std::vector<std::size_t> offset_;    // per node: arena offset
    std::vector<void*> bound_;           // per node: caller device memory, or nullptr
    std::vector<void*> output_bound_;    // per graph output
    std::vector<Launch> launches_;
    std::vector<std::string> sources_;
    double jit_ms_ = 0.0;
};

class HipBackend final : public Backend {
public:
    explicit HipBackend(const HipOptions& options) : options_(options) {}
    const char* name() const override { return "hip"; }
    Result<std::unique_ptr<Executable>> compile(const Graph& graph) override {
        Result<std::unique_ptr<HipExecutable>> exe = compile_for_hip(graph, options_);
        if (!exe.ok()) return exe.error();
        return std::unique_ptr<Executable>(std::move(exe).value());
    }

private:
    HipOptions options_;
};

}  // namespace

Result<std::unique_ptr<HipExecutable>> compile_for_hip(const Graph& graph, const HipOptions& options) {
    Status st = graph.verify();
    if (!st.ok()) return st.error();
    auto exe = std::make_unique<HipExecutableImpl>(graph, options);
    st = exe->init();
    if (!st.ok()) return st.error();
    return std::unique_ptr<HipExecutable>(std::move(exe));
}

Result<std::unique_ptr<Backend>> make_hip_backend(const HipOptions& options) {
    Result<DeviceInfo> dev = query_device(options.device);
    if (!dev.ok()) return Error{"no usable HIP device: " + dev.error().message};
    return std::unique_ptr<Backend>(std::make_unique<HipBackend>(options));
}

}  // namespace minicompiler::hip
