/* Thin C ABI over the HIP runtime and hipRTC.
 *
 * The backend's C++ code reaches the GPU only through these functions, so no
 * C++ source outside this layer and the kernel translation units includes a
 * HIP header. Runtime functions return 0 or a hipError_t value
 * (mchip_error_string describes it); hipRTC functions return 0 or a
 * hiprtcResult value (mchip_rtc_error_string). Handles (streams, events,
 * modules, functions) are opaque pointers.
 *
 * It replaces the reference's direct use of the CUDA runtime, driver and
 * NVRTC in src/cuda/cuda_backend.cpp, src/cuda/kernel_compiler.cpp:24-57 and
 * src/cuda/device_info.cpp:33-73. */
#pragma once

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct mchip_props {
    char name[256];
    char arch[256];
    int cu_count;
    int wave_size;
    int clock_khz;
    int mem_clock_khz;
    int bus_width_bits;
    int l2_bytes;
    size_t total_mem;
    size_t lds_per_block;
    int runtime_version;
    int driver_version;
} mchip_props;

const char* mchip_error_string(int code);

int mchip_device_count(int* count);
int mchip_device_props(int device, mchip_props* props);
int mchip_set_device(int device);
/* The maximum engine clock the runtime reports (kHz). */
int mchip_clock_khz_max(int device, int* khz);
/* "dddd:bb:dd.f", the device's PCI address. */
int mchip_device_pci_bus_id(int device, char* out, int size);

int mchip_malloc(void** ptr, size_t bytes);
int mchip_free(void* ptr);
int mchip_memcpy_htod_async(void* dst, const void* src, size_t bytes, void* stream);
int mchip_memcpy_dtod_async(void* dst, const void* src, size_t bytes, void* stream);
int mchip_memcpy_dtoh(void* dst, const void* src, size_t bytes);
int mchip_memset_async(void* dst, int value, size_t bytes, void* stream);

int mchip_stream_create(void** stream);
int mchip_stream_destroy(void* stream);
int mchip_stream_synchronize(void* stream);
int mchip_device_synchronize(void);

int mchip_event_create(void** event);
int mchip_event_destroy(void* event);
int mchip_event_record(void* event, void* stream);
int mchip_event_synchronize(void* event);
int mchip_event_elapsed_ms(float* ms, void* start, void* stop);

/* hipRTC. On success *code holds the code object (free with mchip_rtc_free);
 * *log always receives the compiler log (may be empty), also malloc'd. */
const char* mchip_rtc_error_string(int code);
int mchip_rtc_compile(const char* source, const char* file_name, const char* const* options, int num_options,
                      char** code, size_t* code_size, char** log);
void mchip_rtc_free(void* p);
/* hiprtcVersion. */
int mchip_rtc_version(int* major, int* minor);

int mchip_module_load(void** module, const void* image);
int mchip_module_unload(void* module);
int mchip_module_function(void** function, void* module, const char* name);
int mchip_module_launch(void* function, unsigned grid, unsigned block, unsigned shared_bytes, void* stream,
                        void** params);
int mchip_module_launch3(void* function, unsigned grid_x, unsigned grid_y, unsigned grid_z, unsigned block,
                         unsigned shared_bytes, void* stream, void** params);
int mchip_occupancy(int* blocks_per_cu, void* function, int block, size_t shared_bytes);

/* Stream capture and replay: hipStreamBeginCapture (thread-local mode);
 * hipStreamEndCapture then hipGraphInstantiate, giving *exec (the graph
 * itself is released; on failure *exec is NULL and capture has ended);
 * hipGraphLaunch; hipGraphExecDestroy. */
int mchip_capture_begin(void* stream);
int mchip_capture_end(void* stream, void** exec);
int mchip_graph_launch(void* exec, void* stream);
int mchip_graph_exec_destroy(void* exec);

#ifdef __cplusplus
}
#endif
