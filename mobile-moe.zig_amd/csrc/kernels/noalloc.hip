// Fixed device scratch for the allocation-free batched QMM entry point
// (mmhip_qmm_dev_noalloc). The array is a file-scope device variable, so it
// exists on every device the library runs on, from module load until the
// process ends, and nothing is allocated or freed per call. Host code never
// passes the array's name to a kernel (on the host it names a stand-in, not
// device memory): noalloc_scratch() looks up each device's own address once,
// with that device current, and callers use that address.
#include "kernels.hpp"

#include <map>
#include <mutex>

namespace mmhip {

static __device__ __align__(256) uint8_t scratch[kNoallocScratchBytes];

hipError_t noalloc_scratch(int device, void** out) {
    static std::mutex mu;
    static std::map<int, void*> per_device;
    std::lock_guard<std::mutex> lk(mu);
    const auto it = per_device.find(device);
    if (it != per_device.end()) {
        *out = it->second;
        return hipSuccess;
    }
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    per_device[device] = p;
    *out = p;
    return hipSuccess;
}

}  // namespace mmhip
