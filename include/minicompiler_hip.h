/* minicompiler_hip.h - the C ABI of the MI355X (gfx950) backend for the
 * minicompiler ML-graph compiler.
 *
 * One shared library, libminicompiler_hip.so, exports these functions with
 * plain pointers and sizes only. Part 1 is exactly the reference's ctypes
 * boundary (bench/capi.cpp), which its Python harness binds
 * (bench/torch_compare.py); part 2 adds what this backend exposes beyond it:
 * compiling from text, in-place device inputs/outputs, graph introspection,
 * the GEMM operator (the reference's launch_matmul, matmul_kernels.hpp:36-59),
 * the kernel generator (codegen.hpp:34-40) and the device memory, stream and
 * event calls a caller needs to drive it without another runtime.
 *
 * Conventions: int-returning calls give 0 on success. Graph-level calls give
 * 1 on failure and record a message readable with mc_last_error() (per
 * thread). Device-level calls (mc_launch_*, mc_device_*, mc_memcpy_*, ...)
 * return the hipError_t value; mc_error_string() describes it. Text-out
 * calls of part 2 write at most `size` bytes including the terminating NUL
 * and return the full length of the text (like snprintf), or -1 on failure;
 * those of part 1 keep the reference's return codes.
 * Handles are not thread-safe; one handle, one thread at a time. */
#ifndef MINICOMPILER_HIP_H
#define MINICOMPILER_HIP_H

#include <stddef.h>

#if defined(__GNUC__)
#define MC_API __attribute__((visibility("default")))
#else
#define MC_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* ---- Part 1: the reference's C interface (bench/capi.cpp) ---------------- */

/* Parses the .mcg file `graph_path` with dim overrides `dims` ("M=64,N=4096"
 * or ""), runs the pass pipeline `passes` ("default", "none" or a list such as
 * "dne,fold") and compiles for `backend`: "hip" (this library's backend) or
 * "none" (passes only; no device is touched, for inspection). Returns NULL and
 * writes a message to `error` on failure. (capi.cpp:62-109) */
MC_API void* mc_compile(const char* graph_path, const char* dims, const char* passes, const char* backend,
                        char* error, int error_size);
MC_API int mc_num_inputs(const void* handle);                   /* capi.cpp:111-113 */
MC_API int mc_num_outputs(const void* handle);                  /* capi.cpp:115-117 */
MC_API long long mc_output_elements(const void* handle, int k); /* capi.cpp:120-123 */
/* Host buffers in graph order; uploads, runs and downloads. (capi.cpp:127-132) */
MC_API int mc_run(void* handle, const float* const* inputs, float* const* outputs);
/* Copies host inputs to the device, where they stay. (capi.cpp:136-147) */
MC_API int mc_upload(void* handle, const float* const* inputs);
/* Launches every kernel on `stream` (a hipStream_t; NULL: the executable's
 * own stream). No copies, no synchronisation. (capi.cpp:150-158) */
MC_API int mc_enqueue(void* handle, void* stream);
/* Waits for the device, then copies outputs to host buffers. (capi.cpp:161-171) */
MC_API int mc_download(void* handle, float* const* outputs);
/* Kernel launches per mc_enqueue, -1 without an executable. (capi.cpp:174-182) */
MC_API int mc_kernel_launches(void* handle);
/* The matmul kernel of each matmul, comma-separated, truncated to `size`.
 * Returns 0, or 1 without an executable (not a length: capi.cpp:184-202). */
MC_API int mc_matmul_kernels(void* handle, char* out, int size);
/* The engine clock in MHz (AMD SMI's current GFX clock of device 0; the
 * reference reads NVML's SM clock), 0 when it cannot be read. AMD SMI's
 * value is the firmware's snapshot, refreshed about once a second.
 * (capi.cpp:204-210) */
MC_API double mc_gpu_sm_clock_mhz(void);
/* mc_gpu_sm_clock_mhz with the snapshot's firmware timestamp in ns (0 when
 * the source has none), so that a sampler keeps one value per snapshot.
 * 0 ok, 1 the clock cannot be read (*mhz = 0). The reference's sampler
 * reads NVML's clock alone (device_info.cpp:14-31, harness.hpp:264-279). */
MC_API int mc_gpu_clock_sample(double* mhz, unsigned long long* stamp_ns);
/* JSON description of device 0 (name, arch, CUs, clocks, bus, peaks) with the
 * `clocks` samples summarised. 0 ok, 1 no device, 2 `out` too small.
 * (capi.cpp:215-231) */
MC_API int mc_gpu_device_json(const double* clocks, int n, char* out, int size);
MC_API void mc_release(void* handle); /* capi.cpp:233-235 */

/* ---- Part 2: extensions ---------------------------------------------------- */

/* mc_compile from graph text, with backend options
 * "matmul=NAME,vectorize=0|1,device=N,epilogue=0|1,tc_convert=0|1,graph=0|1,
 * autotune=0|1,split_fold=0|1,ring=auto|wide|wide8|mid|big|thin|narrow" (graph=1: mc_enqueue captures its
 * launches into a HIP graph once and replays it; rebinding buffers captures
 * again. autotune=1: an auto FP32 matmul's K split and tile configuration
 * are chosen by timing the candidates on the device at compile time, kept
 * per shape for the process and in MINICOMPILER_HIP_CACHE_DIR when set.
 * ring=: the FP32 ring tile configuration of double_buffered / split_k
 * matmuls without autotune, same bits as the planner's) and the elementwise
 * kernel shape "ew_items=N,ew_nt_loads=0|1,ew_nt_stores=0|1,
 * ew_blocks_per_cu=N" (NULL or "" for defaults). */
MC_API void* mc_compile_source(const char* text, const char* dims, const char* passes, const char* backend,
                               const char* options, char* error, int error_size);
/* The message of this thread's last failed call. */
MC_API int mc_last_error(char* out, int size);
MC_API long long mc_input_elements(const void* handle, int k);

/* Device-resident operation (HipExecutable, cuda_backend.hpp:88-104 in the
 * reference, plus in-place binding). Bound pointers must be 16-byte aligned
 * device memory holding the graph's element count; NULL entries keep the
 * executable's own buffer. Bound outputs are written in place by the kernel
 * that computes them. */
MC_API int mc_bind_inputs(void* handle, const void* const* device_inputs);
MC_API int mc_bind_outputs(void* handle, void* const* device_outputs);
MC_API void* mc_input_device_ptr(void* handle, int k);
MC_API void* mc_output_device_ptr(void* handle, int k);
MC_API void* mc_stream(void* handle);
MC_API int mc_synchronize(void* handle);
MC_API double mc_jit_compile_ms(void* handle);
MC_API long long mc_intermediate_bytes(void* handle);
MC_API long long mc_arena_bytes(void* handle);

/* Per-launch timing inside a timed region: mc_profile_start allocates HIP
 * events for `steps` enqueues; each mc_enqueue_profiled then records an event
 * before every launch and after the last one on `stream`; mc_profile_read
 * waits and writes steps x kernel_launches durations in ms (step-major),
 * returning their count. mc_launch_names lists the launches, one per line. */
MC_API int mc_profile_start(void* handle, int steps);
MC_API int mc_enqueue_profiled(void* handle, void* stream);
MC_API int mc_profile_read(void* handle, float* ms, int capacity);
MC_API int mc_launch_names(void* handle, char* out, int size);
/* Launch j of the executable's launch list alone on `stream` (NULL: its own
 * stream), e.g. to time one kernel back to back without events between. */
MC_API int mc_enqueue_launch(void* handle, int j, void* stream);
/* `steps` enqueues in one call, for timing loops with no per-step host
 * work outside the library: step i first binds buffer set i % sets (when
 * sets > 0; set r's inputs at set_inputs[r * num_inputs ...], its outputs
 * at set_outputs[r * num_outputs ...], as mc_bind_inputs / mc_bind_outputs
 * take them; the last set used stays bound), then enqueues the whole step
 * (launch = -1) or only launch `launch` on `stream`. *host_us_per_step
 * (if not NULL) receives the host time per step of the loop. With sets = 0
 * and launch = -1 under option graph_replay, runs of 16 steps replay one
 * captured graph of 16 steps (one hipGraphLaunch per run), the rest the
 * one-step graph. */
MC_API int mc_enqueue_steps(void* handle, int launch, int steps, int sets, const void* const* set_inputs,
                            void* const* set_outputs, void* stream, double* host_us_per_step);
/* The graph nodes each launch computes, launches separated by ';' and nodes
 * by ',' (a matmul with a fused epilogue lists the matmul, then the group). */
MC_API int mc_launch_nodes(void* handle, char* out, int size);

/* The library's seeded generators (random.hpp; fill_uniform is the
 * reference's src/random.cpp:15-26), for callers that build inputs. */
MC_API void mc_fill_uniform(float* out, size_t count, unsigned long long seed, float lo, float hi);
MC_API void mc_fill_normal(float* out, size_t count, unsigned long long seed, double mean, double stddev);

/* Introspection of the compiled graph (after the pipeline). */
/* {"name":..,"nodes":[{"id","op","name","inputs","shape","program"?}],"inputs":[..],"outputs":[..]} */
MC_API int mc_graph_json(const void* handle, char* out, int size);
/* Copies the payload of constant node `node` (count elements). */
MC_API int mc_constant_values(const void* handle, int node, float* out, long long count);
/* Node and op counts after each pipeline stage (input first). */
MC_API int mc_stage_stats_json(const void* handle, char* out, int size);
/* The memory plan: buffer per node, buffer sizes, last uses. */
MC_API int mc_plan_json(const void* handle, int pool_outputs, char* out, int size);
/* Generated HIP source of every elementwise node, in launch order, separated
 * by a line "//----". Works without a device. */
MC_API int mc_kernel_sources(const void* handle, char* out, int size);
/* The graph as `mcc --print` shows it. */
MC_API int mc_print_graph(const void* handle, char* out, int size);

/* The kernel generator (codegen.hpp:34-40): `program` in the printed form,
 * one instruction per line ("r0 = load in0", "r1 = imm 0x3f000000" (bits) or
 * "r1 = imm 0.5", "r2 = mul r0, r1"); `input_shapes` as "[8,64];[64];[]";
 * `out_shape` as "[8,64]"; items_per_lane <= 0: the generator's choice (8
 * for programs of 8 or more ops, else 4). *vectorized receives 1 for
 * 16-byte accesses. */
MC_API int mc_generate_elementwise_kernel(const char* program, const char* input_shapes, const char* out_shape,
                                          int allow_vectorize, int items_per_lane, int* vectorized, char* out,
                                          int size);
/* The matrix-core GEMM whose store applies `program` (its input
 * `acc_input` is the accumulated value; the others are read by access class
 * against `out_shape`), as the executable generates it for a matmul with a
 * fused elementwise consumer, on GEMM body `body`: "two_stage" (or NULL),
 * "ring_big", "ring_wide", "ring_wide8", "ring_mid", "ring_thin", "narrow16",
 * "narrow32", "narrow16x64", "narrow16x32", "narrow64", "bf16", "f16". Works
 * without a device. */
MC_API int mc_generate_gemm_epilogue_kernel(const char* program, int acc_input, const char* input_shapes,
                                            const char* out_shape, int vectorized_operands, const char* body,
                                            char* out, int size);
/* hipRTC-compiles `source` for `arch` (e.g. "gfx950") to a code object with
 * the generator's options; no device needed. Returns 0 or 1; the log goes to
 * `log`. */
MC_API int mc_compile_kernel_source(const char* source, const char* arch, char* log, int log_size);

/* The GEMM operator (launch_matmul, matmul_kernels.hpp:36-59): C[m,n] =
 * A[m,k] B[k,n] row-major fp32 on `stream`. `kernel` is a MatmulKernel value
 * (mc_matmul_kernel_from_name); Auto must be resolved first
 * (mc_resolve_matmul_kernel). Kernels that split K read `splits` and, above
 * 1, `workspace` (mc_matmul_workspace_bytes). Returns a hipError_t value. */
MC_API int mc_launch_matmul(int kernel, const float* a, const float* b, float* c, int m, int n, int k, void* stream,
                            int splits, float* workspace);
/* mc_launch_matmul for double_buffered / split_k with the FP32 ring
 * configuration forced (no counterpart in the reference, whose tiles are
 * fixed; the autotuner picks one, see the `autotune` option): ring_cfg 0 =
 * the planner's own, 1 = wide (128x128 tiles), 2 = mid (64x128), 3 = big
 * (256x256), 4 = thin (32x128), 5 = narrow (32x64 or 16x64 narrow tiles,
 * split_k only, their own accumulation order), 6 = wide8 (128x128 tiles in
 * one 8-wave block per CU). The ring configurations give the same bits.
 * hipErrorInvalidValue when it cannot run the product (K not a multiple of
 * 32, N not of 4, operands not 16-byte aligned) or for other kernels. */
MC_API int mc_launch_matmul_cfg(int kernel, const float* a, const float* b, float* c, int m, int n, int k,
                                void* stream, int splits, float* workspace, int ring_cfg);
/* mc_launch_matmul without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). It has no counterpart in the reference.
 * The split-K partials go to a per-GPU scratch array of mc_noalloc_scratch_bytes()
 * (32 MiB) inside the library, held until the process ends; nothing is
 * allocated per call. A product whose partials (splits x m x n floats for
 * split_k and the tensor-core kernels with splits > 1) exceed it is refused
 * with hipErrorInvalidValue (1) and a message in mc_last_error(). Every call
 * on one GPU shares its array: calls whose executions overlap on one GPU
 * (other streams, other threads) race; calls ordered on one stream do not.
 * Same kernels and bits as mc_launch_matmul with the same `splits`. */
MC_API int mc_launch_matmul_noalloc(int kernel, const float* a, const float* b, float* c, int m, int n, int k,
                                    void* stream, int splits);
MC_API unsigned long long mc_noalloc_scratch_bytes(void);
/* The matrix-core kernels on inputs already stored as bf16 (dtype 1) or fp16
 * (dtype 2); fp32 accumulation and output. */
MC_API int mc_launch_matmul_lowp(int kernel, int dtype, const void* a, const void* b, float* c, int m, int n, int k,
                                 void* stream, int splits, float* workspace);
/* fp32 to bf16 (dtype 1) / fp16 (dtype 2), round to nearest even. */
MC_API int mc_convert_f32(int dtype, const float* in, void* out, size_t count, void* stream);
/* Packed A for the bf16/fp16 kernel. No counterpart in the reference, whose
 * tensor-core kernel (matmul_tensor_core.cu:96-297) stages row-major fp32.
 * A is cut into 256-row bands (the last padded with zero rows) and each band
 * into 32-k steps, each (band, step) block 16 KiB in the kernel's LDS order:
 * element (row, kk) at index (row / 256) 256 k + (kk / 32) 8192 +
 * (row % 256 / 16) 512 + (kk % 32 / 8) 128 + (row % 16) 8 + kk % 8.
 * mc_packed_a16_bytes: its size for an m x k operand; mc_pack_a16: 16-bit
 * row-major A packed; mc_convert_pack_a_f32: fp32 A rounded to bf16 (dtype 1)
 * / fp16 (dtype 2) as mc_convert_f32 rounds and packed (k a multiple of 64,
 * pointers 16-byte aligned); mc_launch_matmul_lowp_packed: the product on
 * packed A and row-major B (K a multiple of 64, N of 8, 16-byte aligned
 * pointers, else hipErrorInvalidValue), the same bits as mc_launch_matmul_lowp
 * on row-major A. Compiled graphs pack the operands they round. */
MC_API long long mc_packed_a16_bytes(int m, int k);
MC_API int mc_pack_a16(const void* a, void* packed, int m, int k, void* stream);
MC_API int mc_convert_pack_a_f32(int dtype, const float* a, void* packed, int m, int k, void* stream);
MC_API int mc_launch_matmul_lowp_packed(int kernel, int dtype, const void* a_packed, const void* b, float* c, int m,
                                        int n, int k, void* stream);
/* c = sum of `splits` partials of `count` floats, fixed order (matmul_kernels.hpp:53-59). */
MC_API int mc_sum_split_partials(const float* partial, float* c, size_t count, int splits, void* stream);
MC_API int mc_split_k_splits(int m, int n, int k, int cu_count, int blocks_per_cu); /* matmul_kernels.hpp:11-17 */
MC_API int mc_matmul_splits(int kernel, int m, int n, int k, int cu_count);         /* matmul_kernels.hpp:23-25 */
/* The K ranges mc_launch_matmul actually runs when given `splits`
 * (16-byte aligned operands, a workspace). No counterpart in the reference,
 * whose split count is exact: here `splits` (and the workspace sized for it)
 * is an upper bound, and split_k's narrow-tile body runs fewer ranges when
 * fewer fill the GPU (256x256x16384 with 64 splits: 8). 1 for kernels that do
 * not split, 0 for invalid sizes. */
MC_API int mc_matmul_k_ranges(int kernel, int m, int n, int k, int splits);
MC_API long long mc_matmul_workspace_bytes(int kernel, int m, int n, int splits);   /* matmul_kernels.hpp:27-30 */
MC_API int mc_resolve_matmul_kernel(int kernel, int m, int n, int k, int cu_count); /* cuda_backend.hpp:45-49 */
MC_API const char* mc_matmul_kernel_name(int kernel);                               /* cuda_backend.hpp:39 */
MC_API int mc_matmul_kernel_from_name(const char* name); /* -1 if unknown (cuda_backend.hpp:41-43) */
MC_API int mc_matmul_supported(int kernel);              /* tensor_core_supported, matmul_kernels.hpp:39-43 */

/* Device memory, streams and events (the thin layer, for callers with no
 * other HIP runtime in the process). */
MC_API int mc_device_count(void);
MC_API int mc_device_malloc(void** ptr, size_t bytes);
MC_API int mc_device_free(void* ptr);
MC_API int mc_memcpy_htod(void* dst, const void* src, size_t bytes);
MC_API int mc_memcpy_dtoh(void* dst, const void* src, size_t bytes);
/* Device-to-device copy enqueued on `stream` (the HIP runtime's own copy,
 * hipMemcpyAsync; no wait). Used as an independent HBM streaming ceiling. */
MC_API int mc_memcpy_dtod_async(void* dst, const void* src, size_t bytes, void* stream);
MC_API int mc_memset(void* dst, int value, size_t bytes);
MC_API int mc_device_synchronize(void);
MC_API int mc_stream_create(void** stream);
MC_API int mc_stream_destroy(void* stream);
MC_API int mc_stream_synchronize(void* stream);
MC_API int mc_event_create(void** event);
MC_API int mc_event_destroy(void* event);
MC_API int mc_event_record(void* event, void* stream);
MC_API int mc_event_elapsed_ms(void* start, void* stop, float* ms);
/* Stream capture into a HIP graph, e.g. to time launches without host
 * launch cost (the reference times its GEMMs from a captured graph,
 * bench/bench_cuda.cpp:445-493): launches enqueued on `stream` between the
 * two calls are recorded, not run; mc_stream_end_capture instantiates them
 * (*graph_exec; NULL on failure, and capture has ended either way). */
MC_API int mc_stream_begin_capture(void* stream);
MC_API int mc_stream_end_capture(void* stream, void** graph_exec);
MC_API int mc_graph_launch(void* graph_exec, void* stream);
MC_API int mc_graph_destroy(void* graph_exec);
MC_API const char* mc_error_string(int code);

#ifdef __cplusplus
}
#endif

#endif /* MINICOMPILER_HIP_H */
