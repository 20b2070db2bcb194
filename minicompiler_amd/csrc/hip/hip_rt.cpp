// Implementation of the thin C ABI (hip_rt.h) over libamdhip64 and libhiprtc.
// Host code only; compiled by the host compiler against the ROCm headers.

#include "hip_rt.h"

#include <hip/hip_runtime_api.h>
#include <hip/hiprtc.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>

extern "C" {

const char* mchip_error_string(int code) { return hipGetErrorString(static_cast<hipError_t>(code)); }

int mchip_device_count(int* count) {
    *count = 0;
    const hipError_t e = hipGetDeviceCount(count);
    if (e == hipErrorNoDevice) {
        *count = 0;
        return hipSuccess;
    }
    return e;
}

int mchip_device_props(int device, mchip_props* out) {
    std::memset(out, 0, sizeof *out);
    hipDeviceProp_t p;
    hipError_t e = hipGetDeviceProperties(&p, device);
    if (e != hipSuccess) return e;
    std::snprintf(out->name, sizeof out->name, "%s", p.name);
    std::snprintf(out->arch, sizeof out->arch, "%s", p.gcnArchName);
    out->cu_count = p.multiProcessorCount;
    out->wave_size = p.warpSize;
    out->total_mem = p.totalGlobalMem;
    out->lds_per_block = p.sharedMemPerBlock;
    out->l2_bytes = p.l2CacheSize;
    if ((e = hipDeviceGetAttribute(&out->clock_khz, hipDeviceAttributeClockRate, device)) != hipSuccess) return e;
    if ((e = hipDeviceGetAttribute(&out->mem_clock_khz, hipDeviceAttributeMemoryClockRate, device)) != hipSuccess)
        return e;
    if ((e = hipDeviceGetAttribute(&out->bus_width_bits, hipDeviceAttributeMemoryBusWidth, device)) != hipSuccess)
        return e;
    if ((e = hipRuntimeGetVersion(&out->runtime_version)) != hipSuccess) return e;
    return hipDriverGetVersion(&out->driver_version);
}

int mchip_set_device(int device) { return hipSetDevice(device); }

int mchip_clock_khz_max(int device, int* khz) {
    return hipDeviceGetAttribute(khz, hipDeviceAttributeClockRate, device);
}

int mchip_device_pci_bus_id(int device, char* out, int size) { return hipDeviceGetPCIBusId(out, size, device); }

int mchip_malloc(void** ptr, size_t bytes) { return hipMalloc(ptr, bytes); }
int mchip_free(void* ptr) { return hipFree(ptr); }

int mchip_memcpy_htod_async(void* dst, const void* src, size_t bytes, void* stream) {
    return hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, static_cast<hipStream_t>(stream));
}
int mchip_memcpy_dtod_async(void* dst, const void* src, size_t bytes, void* stream) {
    return hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, static_cast<hipStream_t>(stream));
}
int mchip_memcpy_dtoh(void* dst, const void* src, size_t bytes) {
    return hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost);
}
int mchip_memset_async(void* dst, int value, size_t bytes, void* stream) {
    return hipMemsetAsync(dst, value, bytes, static_cast<hipStream_t>(stream));
}

int mchip_stream_create(void** stream) {
    // Default priority: streams here never carry a priority.
    return hipStreamCreateWithFlags(reinterpret_cast<hipStream_t*>(stream), hipStreamNonBlocking);
}
int mchip_stream_destroy(void* stream) { return hipStreamDestroy(static_cast<hipStream_t>(stream)); }
int mchip_stream_synchronize(void* stream) { return hipStreamSynchronize(static_cast<hipStream_t>(stream)); }
int mchip_device_synchronize(void) { return hipDeviceSynchronize(); }

int mchip_event_create(void** event) { return hipEventCreate(reinterpret_cast<hipEvent_t*>(event)); }
int mchip_event_destroy(void* event) { return hipEventDestroy(static_cast<hipEvent_t>(event)); }
int mchip_event_record(void* event, void* stream) {
    return hipEventRecord(static_cast<hipEvent_t>(event), static_cast<hipStream_t>(stream));
}
int mchip_event_synchronize(void* event) { return hipEventSynchronize(static_cast<hipEvent_t>(event)); }
int mchip_event_elapsed_ms(float* ms, void* start, void* stop) {
    return hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop));
}

const char* mchip_rtc_error_string(int code) { return hiprtcGetErrorString(static_cast<hiprtcResult>(code)); }

int mchip_rtc_compile(const char* source, const char* file_name, const char* const* options, int num_options,
                      char** code, size_t* code_size, char** log) {
    *code = nullptr;
    *code_size = 0;
    *log = nullptr;
    hiprtcProgram prog = nullptr;
    hiprtcResult r = hiprtcCreateProgram(&prog, source, file_name, 0, nullptr, nullptr);
    if (r != HIPRTC_SUCCESS) return r;
    const hiprtcResult compiled = hiprtcCompileProgram(prog, num_options, const_cast<const char**>(options));
    size_t log_size = 0;
    if (hiprtcGetProgramLogSize(prog, &log_size) == HIPRTC_SUCCESS) {
        *log = static_cast<char*>(std::calloc(log_size + 1, 1));
        if (*log && log_size > 0) hiprtcGetProgramLog(prog, *log);
    }
    r = compiled;
    if (r == HIPRTC_SUCCESS) r = hiprtcGetCodeSize(prog, code_size);
    if (r == HIPRTC_SUCCESS) {
        *code = static_cast<char*>(std::malloc(*code_size));
        r = *code ? hiprtcGetCode(prog, *code) : HIPRTC_ERROR_OUT_OF_MEMORY;
    }
    hiprtcDestroyProgram(&prog);
    return r;
}

void mchip_rtc_free(void* p) { std::free(p); }
int mchip_rtc_version(int* major, int* minor) { return hiprtcVersion(major, minor); }

int mchip_module_load(void** module, const void* image) {
    return hipModuleLoadData(reinterpret_cast<hipModule_t*>(module), image);
}
int mchip_module_unload(void* module) { return hipModuleUnload(static_cast<hipModule_t>(module)); }
int mchip_module_function(void** function, void* module, const char* name) {
    return hipModuleGetFunction(reinterpret_cast<hipFunction_t*>(function), static_cast<hipModule_t>(module), name);
}
int mchip_module_launch(void* function, unsigned grid, unsigned block, unsigned shared_bytes, void* stream,
                        void** params) {
    return hipModuleLaunchKernel(static_cast<hipFunction_t>(function), grid, 1, 1, block, 1, 1, shared_bytes,
                                 static_cast<hipStream_t>(stream), params, nullptr);
}
int mchip_module_launch3(void* function, unsigned grid_x, unsigned grid_y, unsigned grid_z, unsigned block,
                         unsigned shared_bytes, void* stream, void** params) {
    return hipModuleLaunchKernel(static_cast<hipFunction_t>(function), grid_x, grid_y, grid_z, block, 1, 1,
                                 shared_bytes, static_cast<hipStream_t>(stream), params, nullptr);
}
int mchip_occupancy(int* blocks_per_cu, void* function, int block, size_t shared_bytes) {
    return hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(blocks_per_cu, static_cast<hipFunction_t>(function),
                                                              block, shared_bytes);
}

int mchip_capture_begin(void* stream) {
    return hipStreamBeginCapture(static_cast<hipStream_t>(stream), hipStreamCaptureModeThreadLocal);
}
int mchip_capture_end(void* stream, void** exec) {
    *exec = nullptr;
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamEndCapture(static_cast<hipStream_t>(stream), &graph);
    if (e != hipSuccess) return e;
    hipGraphExec_t x = nullptr;
    e = hipGraphInstantiate(&x, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (e != hipSuccess) return e;
    *exec = x;
    return hipSuccess;
}
int mchip_graph_launch(void* exec, void* stream) {
    return hipGraphLaunch(static_cast<hipGraphExec_t>(exec), static_cast<hipStream_t>(stream));
}
int mchip_graph_exec_destroy(void* exec) { return hipGraphExecDestroy(static_cast<hipGraphExec_t>(exec)); }

}  // extern "C"
