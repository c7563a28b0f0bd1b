// scratch.hip - library-held device scratch for the entry point that
// allocates nothing (jules_hip_w8a16_gemm_bias_act_noalloc).
//
// `scratch` is a file-scope device array: every GPU the library runs on holds
// its own copy, at its own address, from module load to process exit.  In
// host code the name `scratch` is only a host-side handle, not a device
// address; the device address is looked up once per device with
// hipGetSymbolAddress (with that device current) and kept, and only that
// address is ever handed to a kernel.
#include <mutex>

#include "launch.hpp"

// 8 MiB of split-K partials (8 splits x 64 column tiles of 16 KiB: N up to
// 16384 at any K), then 4 KiB holding the per-tile arrival counters (zero at
// load; every call leaves them at zero)
static constexpr size_t kPartialBytes = size_t(8) << 20;
static constexpr size_t kScratchBytes = kPartialBytes + 4096;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace jh {
namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];  // device address of `scratch` per device
}  // namespace

size_t static_scratch_bytes() { return kScratchBytes; }
size_t static_scratch_partial_bytes() { return kPartialBytes; }

hipError_t static_scratch(void** ptr) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        g_scratch_ptr[dev] = p;
    }
    *ptr = g_scratch_ptr[dev];
    return hipSuccess;
}

}  // namespace jh
