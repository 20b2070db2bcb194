// The GEMM operator for callers that cannot allocate device memory (code
// under HIP graph capture, tight serving loops, harnesses that forbid
// hipMalloc): mchip_launch_matmul with the split-K partials kept in a
// file-scope device array instead of a caller workspace.
//
// The array is `scratch`, kScratchBytes long, one copy per GPU, held from
// the library's first use on that GPU until the process ends. Host code never
// passes the array's name to a kernel (on the host it is only a stand-in for
// the device symbol): the first call on a device asks the runtime for the
// array's device address on that device (hipGetSymbolAddress, with that
// device current) and keeps it; every later call on the device uses the kept
// address. Calls on one GPU share the array, so calls whose executions
// overlap on one GPU (different streams, or different threads) race on it;
// calls ordered on one stream do not. Nothing in the array has to start at
// any value: each split writes every element of its partial before the
// fixed-order sum reads it.

#include "matmul.h"

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstddef>
#include <mutex>

static constexpr std::size_t kScratchBytes = std::size_t{32} << 20;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kMaxDevices = 64;

std::atomic<void*> g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mu;

// The current device's address of `scratch`, looked up once per device.
hipError_t scratch_address(void** out) {
    *out = nullptr;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
    if (p == nullptr) {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
        if (p == nullptr) {
            e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (e != hipSuccess) return e;
            if (p == nullptr) return hipErrorInvalidSymbol;
            g_scratch_ptr[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return hipSuccess;
}

}  // namespace

extern "C" unsigned long long mchip_noalloc_scratch_bytes(void) { return kScratchBytes; }

extern "C" unsigned long long mchip_noalloc_required_bytes(int kernel, int m, int n, int splits) {
    // The partials of a K-splitting kernel (split_k and the tensor-core
    // rungs: MatmulKernel values 7..10): splits x m x n floats.
    if (splits <= 1 || kernel < 7 || kernel > 10 || m < 1 || n < 1) return 0;
    return static_cast<unsigned long long>(splits) * static_cast<unsigned long long>(m) *
           static_cast<unsigned long long>(n) * sizeof(float);
}

extern "C" int mchip_launch_matmul_noalloc(int kernel, const float* a, const float* b, float* c, int m, int n, int k,
                                           void* stream, int splits) {
    if (m < 1 || n < 1 || k < 1 || splits < 1) return hipErrorInvalidValue;
    const unsigned long long need = mchip_noalloc_required_bytes(kernel, m, n, splits);
    if (need > kScratchBytes) return hipErrorInvalidValue;
    float* workspace = nullptr;
    if (need > 0) {
        void* p = nullptr;
        const hipError_t e = scratch_address(&p);
        if (e != hipSuccess) return e;
        workspace = static_cast<float*>(p);
    }
    return mchip_launch_matmul(kernel, a, b, c, m, n, k, stream, splits, workspace);
}
