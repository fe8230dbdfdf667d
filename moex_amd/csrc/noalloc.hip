// Device scratch of moex_attn_decode_noalloc (include/moex_attn.h): a file-scope device array, so that entry point
// needs no hipMalloc. Each device that loads the library holds its own copy at its own address until the process
// ends; the host finds that address once per device with hipGetSymbolAddress and passes it to the kernels (the
// array's name in host code is only a host-side stand-in, not a device address).
#include <hip/hip_runtime.h>
#include <mutex>
#include "common.hpp"

namespace moex {

namespace {
__device__ __align__(256) unsigned char scratch[MOEX_NOALLOC_SCRATCH_BYTES];

constexpr int MAX_DEV = 64;
std::mutex g_mu;
void* g_ptr[MAX_DEV];  // per device: the address of its copy of scratch
}  // namespace

float* noalloc_scratch() {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) {
        report(e, __FILE__, __LINE__);
        return nullptr;
    }
    if (dev < 0 || dev >= MAX_DEV) {
        report(hipErrorInvalidDevice, __FILE__, __LINE__);
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_mu);
    if (!g_ptr[dev]) {  // first call on this device, which is current here
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            report(e != hipSuccess ? e : hipErrorInvalidSymbol, __FILE__, __LINE__);
            return nullptr;
        }
        g_ptr[dev] = p;
    }
    return static_cast<float*>(g_ptr[dev]);
}

}  // namespace moex
