#pragma once

// The HIP backend for AMD Instinct MI355X (gfx950 / CDNA4). It takes the
// place of the reference's CUDA backend behind the same Backend/Executable
// interface (reference: include/minicompiler/cuda/cuda_backend.hpp:20-107).
// This header includes no HIP header: every HIP call goes through the
// library's thin C-ABI layer.

#include "minicompiler/graph.hpp"
#include "minicompiler/result.hpp"
#include "minicompiler/runtime/backend.hpp"

#include <cstddef>
#include <memory>
#include <string>
#include <vector>

namespace minicompiler::hip {

// The matmul kernels, same names as the reference's MatmulKernel
// (cuda_backend.hpp:20-37). On CDNA4:
//   Naive, Tiled, RegisterTiled128, RegisterTiled64: FP32 on the vector ALU
//     (one output per lane; 32x32 LDS tiles; 128x128 and 64x64 tiles with an
//     8x8 / 4x4 register block per lane).
//   Vectorized: 128x128 tiles staged in LDS with 16-byte global loads, the
//     products on the FP32 matrix cores (v_mfma_f32_32x32x2_f32), one LDS stage.
//   DoubleBuffered: Vectorized with the next tile's loads in flight while
//     the current one is multiplied: where K % 32 = 0 and N % 4 = 0, a ring
//     of 2 or 4 LDS stages filled by direct global -> LDS loads, persistent
//     blocks in XCD order, 256x256 or 128x128 tiles; otherwise two LDS
//     stages. The same arithmetic as Vectorized, bit for bit.
//   SplitK: DoubleBuffered with K split into whole 32-wide steps and a
//     deterministic fixed-order reduction of the partial products.
//   TensorCoreBf16 / TensorCoreF16: inputs rounded to nearest-even into
//     bf16 / fp16 while they are staged in LDS, products on the bf16 / fp16
//     matrix cores (v_mfma_f32_16x16x32_{bf16,f16}), FP32 accumulation, split-K
//     where SplitK splits.
//   TensorCoreTf32: gfx950 has no xf32 matrix instruction; compiling a graph
//     with it fails, naming the kernel and the device.
enum class MatmulKernel {
    Auto,
    Naive,
    Tiled,
    RegisterTiled128,
    RegisterTiled64,
    Vectorized,
    DoubleBuffered,
    SplitK,
    TensorCoreTf32,
    TensorCoreBf16,
    TensorCoreF16,
};

const char* matmul_kernel_name(MatmulKernel kernel);
Result<MatmulKernel> matmul_kernel_from_name(const std::string& name);

// Auto becomes SplitK when split_k_splits() divides K for this shape on
// `cu_count` CUs, DoubleBuffered otherwise; every other kernel is returned
// unchanged (reference: cuda_backend.cpp:43-49).
MatmulKernel resolve_matmul_kernel(MatmulKernel kernel, int m, int n, int k, int cu_count);

struct HipOptions {
    int device = 0;
    MatmulKernel matmul = MatmulKernel::Auto;
    // 16-byte loads and stores in elementwise kernels when the layout allows.
    bool vectorize = true;
    // Elementwise kernel shape: vectors (or floats) each lane has in flight
    // per loop step, non-temporal hints on the streaming loads and stores,
    // and the grid's blocks per CU (more than fit at once run in turn;
    // 0: 64, so in practice one loop step per block), capped by the work.
    unsigned elementwise_items = 0;  // 0: by the program (8 for 8 or more ops, else 4)
    bool nontemporal_loads = true;
    bool nontemporal_stores = true;
    unsigned elementwise_blocks_per_cu = 0;
    // Apply a fused elementwise group that consumes a matmul's product in
    // the store of an FP32 matrix-core GEMM (one kernel instead of two), when
    // the memory plan makes that safe.
    bool fuse_epilogue = true;
    // Tensor-core matmuls (bf16 / fp16) in a compiled graph: round the fp32
    // operands to 16 bits into workspace first (constants once, at compile
    // time), then run the 256x256-tile kernel on them, when the shape allows
    // (K a multiple of 64, N a multiple of 8). The rounding and the
    // accumulation order are those of the staging kernel with K unsplit, so
    // results match that kernel bit for bit. Off: the staging kernel rounds
    // while it stages (and splits K where SplitK would).
    bool convert_tensor_core_operands = true;
    // enqueue() captures its launches into a HIP graph the first time and
    // replays that graph afterwards (one submission instead of one per
    // kernel); binding other buffers captures again. The graph holds kernel
    // launches and, for graph outputs that are inputs or constants, copies;
    // no memsets. The stream must be one that can be captured (not the
    // legacy null stream). enqueue_launch and enqueue_with_events launch
    // directly.
    bool graph_replay = false;
    // An Auto FP32 matmul's K split and ring tile configuration are chosen by
    // timing the candidates on the device at compile time (double_buffered
    // unsplit or split_k with 2, 4, ... splits, on 128x128, 64x128 or 32x128
    // tiles) instead of by the split rule and the planner. Decisions are kept
    // per device and shape for the process, and in MINICOMPILER_HIP_CACHE_DIR
    // when set. Different split counts round differently (within the FP32
    // GEMM bound); the tile configuration does not change the bits.
    bool autotune = false;
    // split_k matmuls on the ring or narrow FP32 bodies add their K splits'
    // partials inside the GEMM launch: the last block to finish a split of a
    // C tile adds the tile's partials in split order (the same bits as the
    // separate sum) and stores C through any fused epilogue; per-tile arrival
    // counters live in the arena, zeroed once at compile time. Off (the
    // default): a separate sum launch, as the C ABI's mc_launch_matmul does.
    // Measured on an MI355X (graph-timed, operands past the MALL), the fold
    // is the slower: 16x4096x4096 18.0 us against 17.0, 256x256x16384 30.5
    // against 28.1, 1024^3 61 against 28 (one CU per tile reads the tile's
    // partials with device-scope loads, at memory latency).
    bool split_fold = false;
    // The FP32 ring tile configuration of double_buffered / split_k matmuls
    // without autotune (MCHIP_RING_*: 0 the planner's own, 1 wide 128x128,
    // 2 mid 64x128, 3 big 256x256, 4 thin 32x128, 5 narrow tiles for split_k,
    // 6 wide8: 128x128 in one 8-wave block per CU). The ring configurations
    // give the same bits as each other.
    int ring_config = 0;
};

// What the device reports (hipGetDeviceProperties / hipDeviceGetAttribute).
struct DeviceInfo {
    std::string name;           // marketing name
    std::string arch;           // gcnArchName, e.g. "gfx950:sramecc+:xnack-"
    int cu_count = 0;
    int wave_size = 0;
    double clock_mhz = 0;       // max engine clock the runtime reports
    double mem_clock_mhz = 0;
    int bus_width_bits = 0;
    std::size_t total_memory = 0;
    std::size_t l2_bytes = 0;
    std::size_t lds_bytes_per_block = 0;
    int runtime_version = 0;
    int driver_version = 0;

    // Transfers per reported memory clock x memory clock x bus width. The
    // reference's formula counts two transfers (cuda_backend.hpp:73-76); the
    // HIP runtime reports CDNA's HBM clock at a quarter of the per-pin data
    // rate (MI355X: 2000 MHz for 8 Gb/s HBM3E on 8192 bits, 8.19 TB/s, the
    // published 8 TB/s), so four here.
    double peak_bandwidth_gbs() const { return 4.0 * mem_clock_mhz * 1e6 * bus_width_bits / 8.0 / 1e9; }
    // CDNA4 per CU and clock: 256 FP32 FLOP (matrix cores, or packed vector
    // FMA), 4096 dense bf16/fp16 FLOP on the matrix cores.
    double peak_fp32_gflops(double clock) const { return 256.0 * cu_count * clock * 1e6 / 1e9; }
    double peak_bf16_gflops(double clock) const { return 4096.0 * cu_count * clock * 1e6 / 1e9; }
};

Result<DeviceInfo> query_device(int device = 0);

// The engine clock in MHz at the power-management firmware's last refresh
// of its metrics (about once a second), or 0 when the runtime cannot tell.
double current_clock_mhz(int device = 0);
// The same, with the refresh's firmware timestamp in ns (0 when the source
// has none): reads with the same stamp are the same snapshot. False, with 0
// MHz, when the clock cannot be read.
bool current_clock_sample(int device, double* mhz, unsigned long long* stamp_ns);

// A graph compiled for the GPU. Every device allocation is one arena taken at
// compile time: pooled intermediates and outputs at the memory plan's
// offsets, graph inputs, constants (uploaded once) and split-K workspaces.
class HipExecutable : public Executable {
public:
    // Copies host inputs into the arena; returns once they are resident.
    virtual Status upload_inputs(const std::vector<const float*>& host_inputs) = 0;
    // Launches every kernel in order on `stream` (a hipStream_t; nullptr: the
    // executable's own stream). No copies, no synchronisation.
    virtual Status enqueue(void* stream = nullptr) = 0;
    // enqueue() with events[j] recorded before launch j and events[launches]
    // after the last one (kernel_launches() + 1 hipEvent_t handles).
    virtual Status enqueue_with_events(void* stream, void* const* events) = 0;
    // Launch j of the list alone (for timing one kernel back to back).
    virtual Status enqueue_launch(std::size_t j, void* stream = nullptr) = 0;
    // `count` enqueues back to back on the same buffers. With graph_replay,
    // runs of kGraphSteps steps replay one captured graph of that many
    // steps (one submission per run instead of per step); the rest replay
    // the one-step graph.
    virtual Status enqueue_steps(int count, void* stream = nullptr) = 0;
    static constexpr int kGraphSteps = 16;
    virtual Status synchronize() = 0;
    // Waits for the device, then copies the outputs to the host.
    virtual Status download_outputs(const std::vector<float*>& host_outputs) = 0;

    // Caller-owned device memory for inputs / outputs (nullptr entries keep
    // the arena's buffer). Bound outputs are written in place by the kernel
    // that computes them, with no copy. Pointers must be 16-byte aligned.
    virtual Status bind_inputs(const std::vector<const void*>& device_inputs) = 0;
    virtual Status bind_outputs(const std::vector<void*>& device_outputs) = 0;
    virtual void* input_device_ptr(std::size_t k) const = 0;
    virtual void* output_device_ptr(std::size_t k) const = 0;
    // The executable's own stream (a hipStream_t).
    virtual void* stream() const = 0;

    virtual std::size_t kernel_launches() const = 0;
    virtual std::vector<std::string> kernel_sources() const = 0;
    // One label per launch: "matmul <kernel> MxNxK" or "<op> <node> f32[...]".
    virtual std::vector<std::string> launch_names() const = 0;
    // The graph nodes each launch computes (a fused matmul: the matmul and
    // its epilogue group).
    virtual std::vector<std::vector<NodeId>> launch_nodes() const = 0;
    virtual std::vector<MatmulKernel> matmul_kernels() const = 0;
    virtual double jit_compile_ms() const = 0;
    virtual std::size_t arena_bytes() const = 0;
};

Result<std::unique_ptr<HipExecutable>> compile_for_hip(const Graph& graph, const HipOptions& options = {});
Result<std::unique_ptr<Backend>> make_hip_backend(const HipOptions& options = {});

}  // namespace minicompiler::hip
