// Device queries (replaces the reference's src/cuda/device_info.cpp:33-66,
// which read CUDA properties; the live clock is in engine_clock.cpp).

#include "hip_rt.h"
#include "minicompiler/hip/hip_backend.hpp"

namespace minicompiler::hip {

Result<DeviceInfo> query_device(int device) {
    int count = 0;
    int rc = mchip_device_count(&count);
    if (rc != 0) return Error{std::string("hipGetDeviceCount: ") + mchip_error_string(rc)};
    if (device < 0 || device >= count) {
        return Error{"no HIP device " + std::to_string(device) + " (" + std::to_string(count) + " present)"};
    }
    mchip_props p;
    rc = mchip_device_props(device, &p);
    if (rc != 0) return Error{std::string("hipGetDeviceProperties: ") + mchip_error_string(rc)};
    DeviceInfo info;
    info.name = p.name;
    info.arch = p.arch;
    info.cu_count = p.cu_count;
    info.wave_size = p.wave_size;
    info.clock_mhz = p.clock_khz / 1000.0;
    info.mem_clock_mhz = p.mem_clock_khz / 1000.0;
    info.bus_width_bits = p.bus_width_bits;
    info.total_memory = p.total_mem;
    info.l2_bytes = static_cast<std::size_t>(p.l2_bytes);
    info.lds_bytes_per_block = p.lds_per_block;
    info.runtime_version = p.runtime_version;
    info.driver_version = p.driver_version;
    return info;
}

}  // namespace minicompiler::hip
