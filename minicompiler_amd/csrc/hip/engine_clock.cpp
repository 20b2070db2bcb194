// The live engine (GFX) clock of a device, read through AMD SMI, the
// counterpart of the reference's NVML clock query
// (src/cuda/device_info.cpp:14-31, 68-73). HIP itself reports only the
// maximum engine clock.
//
// libamd_smi is loaded at run time (dlopen), so the library has no link-time
// dependency on it; without it, or without a metrics table for the device,
// the clock reads 0 ("cannot tell"), as the reference's does without NVML.
// The device is matched to its AMD SMI handle by PCI address, because the
// two may number devices differently (the reference matches NVML the same
// way). The value is the gpu_metrics table's current GFX clock: the mean of
// the per-XCC current clocks when the table has them (MI300-class parts),
// else its single current clock, else the 1-second average AMD SMI reports.
//
// The power-management firmware refreshes that table about once a second
// (on an MI355X its timestamp advanced in steps of 1.000 s, and AMD SMI's
// clock query returned the same snapshot): a read is the clock at the last
// refresh, not at the moment of the call. current_clock_sample also returns
// the snapshot's firmware timestamp, so a caller can keep one value per
// snapshot.

#include "hip_rt.h"
#include "minicompiler/hip/hip_backend.hpp"

#include <amd_smi/amdsmi.h>
#include <dlfcn.h>

#include <cstdio>
#include <map>
#include <mutex>

namespace minicompiler::hip {

namespace {

struct AmdSmi {
    decltype(&amdsmi_init) init = nullptr;
    decltype(&amdsmi_get_processor_handle_from_bdf) handle_from_bdf = nullptr;
    decltype(&amdsmi_get_gpu_metrics_info) metrics = nullptr;
    decltype(&amdsmi_get_clock_info) clock_info = nullptr;
    bool ok = false;
};

const AmdSmi& amdsmi() {
    static AmdSmi smi;
    static std::once_flag once;
    std::call_once(once, [] {
        void* lib = dlopen("libamd_smi.so", RTLD_NOW | RTLD_LOCAL);
        if (lib == nullptr) lib = dlopen("/opt/rocm/lib/libamd_smi.so", RTLD_NOW | RTLD_LOCAL);
        if (lib == nullptr) return;
        smi.init = reinterpret_cast<decltype(smi.init)>(dlsym(lib, "amdsmi_init"));
        smi.handle_from_bdf = reinterpret_cast<decltype(smi.handle_from_bdf)>(
            dlsym(lib, "amdsmi_get_processor_handle_from_bdf"));
        smi.metrics = reinterpret_cast<decltype(smi.metrics)>(dlsym(lib, "amdsmi_get_gpu_metrics_info"));
        smi.clock_info = reinterpret_cast<decltype(smi.clock_info)>(dlsym(lib, "amdsmi_get_clock_info"));
        smi.ok = smi.init && smi.handle_from_bdf && smi.init(AMDSMI_INIT_AMD_GPUS) == AMDSMI_STATUS_SUCCESS;
    });
    return smi;
}

// The AMD SMI handle of HIP device `device`, looked up once.
bool processor_of(int device, amdsmi_processor_handle* out) {
    static std::mutex mu;
    static std::map<int, amdsmi_processor_handle> known;
    const AmdSmi& smi = amdsmi();
    if (!smi.ok) return false;
    std::lock_guard<std::mutex> lock(mu);
    const auto it = known.find(device);
    if (it != known.end()) {
        *out = it->second;
        return it->second != nullptr;
    }
    amdsmi_processor_handle h = nullptr;
    char bus[64] = {};
    unsigned domain = 0, bus_no = 0, dev_no = 0, fn = 0;
    if (mchip_device_pci_bus_id(device, bus, sizeof bus) == 0 &&
        std::sscanf(bus, "%x:%x:%x.%x", &domain, &bus_no, &dev_no, &fn) == 4) {
        amdsmi_bdf_t bdf{};
        bdf.domain_number = domain;
        bdf.bus_number = bus_no;
        bdf.device_number = dev_no;
        bdf.function_number = fn;
        if (smi.handle_from_bdf(bdf, &h) != AMDSMI_STATUS_SUCCESS) h = nullptr;
    }
    known[device] = h;
    *out = h;
    return h != nullptr;
}

bool valid_mhz(unsigned v) { return v != 0 && v != 0xFFFF; }

}  // namespace

bool current_clock_sample(int device, double* mhz, unsigned long long* stamp_ns) {
    *mhz = 0.0;
    *stamp_ns = 0;
    amdsmi_processor_handle h = nullptr;
    if (!processor_of(device, &h)) return false;
    const AmdSmi& smi = amdsmi();
    if (smi.metrics) {
        amdsmi_gpu_metrics_t m{};
        if (smi.metrics(h, &m) == AMDSMI_STATUS_SUCCESS) {
            double sum = 0.0;
            int n = 0;
            for (unsigned v : m.current_gfxclks) {
                if (valid_mhz(v)) {
                    sum += v;
                    ++n;
                }
            }
            *stamp_ns = static_cast<unsigned long long>(m.firmware_timestamp) * 10;  // 10 ns units
            if (n > 0) {
                *mhz = sum / n;
                return true;
            }
            if (valid_mhz(m.current_gfxclk)) {
                *mhz = m.current_gfxclk;
                return true;
            }
            *stamp_ns = 0;
        }
    }
    if (smi.clock_info) {
        amdsmi_clk_info_t info{};
        if (smi.clock_info(h, AMDSMI_CLK_TYPE_GFX, &info) == AMDSMI_STATUS_SUCCESS && info.clk > 0) {
            *mhz = info.clk;
            return true;
        }
    }
    return false;
}

double current_clock_mhz(int device) {
    double mhz = 0.0;
    unsigned long long stamp = 0;
    current_clock_sample(device, &mhz, &stamp);
    return mhz;
}

}  // namespace minicompiler::hip
