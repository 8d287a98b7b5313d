// Measurement utility for bench.py (not part of libmmhip's ABI): a plain
// streaming read of a device buffer, the STREAM-style ceiling the GEMV rates
// are compared with, and the kernel of known size that calibrates the
// FETCH_SIZE counter. Each thread keeps four independent 16-byte loads in
// flight per iteration (non-temporal: read once) and folds them into a
// checksum, which one lane per workgroup stores so the loads are not dead.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr int kThreads = 512;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kThreads) void read_kernel(const u32x4* __restrict__ p, uint64_t n16,
                                                        uint32_t* __restrict__ sink) {
    const uint64_t stride = (uint64_t)gridDim.x * kThreads;
    uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
    uint32_t acc = 0;
    for (; i + 3 * stride < n16; i += 4 * stride) {
        u32x4 v[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = __builtin_nontemporal_load(p + i + k * stride);
#pragma unroll
        for (int k = 0; k < 4; ++k) acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
    }
    for (; i < n16; i += stride) {
        const u32x4 v = __builtin_nontemporal_load(p + i);
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    // Any lane's value is as good as another's: the store only keeps the loads alive.
    if (threadIdx.x == 0) sink[blockIdx.x] = acc;
}

}  // namespace

extern "C" {

// Reads `bytes` (a multiple of 16) from `buf` once; `sink` must hold
// `blocks` uint32 values. Asynchronous on `stream`.
int mmbench_read(const void* buf, uint64_t bytes, void* sink, uint32_t blocks, void* stream) {
    if (!buf || !sink || bytes % 16 || blocks == 0) return -2;
    read_kernel<<<blocks, kThreads, 0, (hipStream_t)stream>>>((const u32x4*)buf, bytes / 16, (uint32_t*)sink);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

}  // extern "C"
