// noalloc.hip -- the GEMM entry point that allocates nothing
// (t0_gemm_noalloc).  Compiled by hipcc as a host + device translation unit:
// the scratch array below is a file-scope device variable of this library,
// one copy per GPU, present for the life of the process.  Host code never
// uses the array's name as an address: each device's address is resolved
// once (hipGetSymbolAddress, at runtime creation) and that pointer is what
// the kernels receive.
#include <hip/hip_runtime.h>

#include <mutex>

#include "internal.hpp"

static __device__ __align__(256) uint8_t scratch[T0_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices];   // scratch's address on each device, once resolved
}  // namespace

// With `device` current: resolve this device's copy of the scratch array.
extern "C" int t0h_noalloc_setup(int device) {
    if (device < 0 || device >= kMaxDevices) return t0h::fail(T0_ERR_NO_DEVICE, "device %d out of range", device);
    std::lock_guard<std::mutex> g(g_mu);
    if (g_ptr[device]) return T0_OK;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
        return t0h::fail(T0_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", device, hipGetErrorString(e));
    g_ptr[device] = p;
    return T0_OK;
}

extern "C" int t0_gemm_noalloc(t0_runtime* rt, const t0_gemm_config* cfg, const t0_gemm_desc* d) {
    if (!rt || !d) return t0h::fail(T0_ERR_INVALID, "null argument");
    const int dev = t0h::runtime_device(rt);
    void* p = nullptr;
    {
        std::lock_guard<std::mutex> g(g_mu);
        if (dev >= 0 && dev < kMaxDevices) p = g_ptr[dev];
    }
    if (!p) return t0h::fail(T0_ERR_INVALID, "no-allocation scratch not set up on device %d", dev);
    return t0h::gemm_with_scratch(rt, cfg, d, p, T0_NOALLOC_SCRATCH_BYTES);
}
