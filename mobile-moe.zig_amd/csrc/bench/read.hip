// Measurement utility for bench.py (not part of libmmhip's ABI): a plain
// streaming read of a device buffer, the STREAM-style ceiling the GEMV rates
// are compared with, and the kernel of known size that calibrates the
// FETCH_SIZE counter. Short-lived waves: each thread issues four independent
// 16-byte non-temporal loads (i, i + T, i + 2T, i + 3T for T threads) and
// exits; on MI355X this reads 6.8 TB/s where a grid-stride loop over the same
// loads reaches 6.45 TB/s. The loads are kept alive by a store that a
// zero-filled buffer never triggers.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

constexpr int kThreads = 256;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kThreads) void read_kernel(const u32x4* __restrict__ p, uint64_t n16, uint64_t n_thr,
                                                        uint32_t* __restrict__ sink) {
    const uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
    uint32_t acc = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint64_t j = i + k * n_thr;
        if (j < n16) {
            const u32x4 v = __builtin_nontemporal_load(p + j);
            acc ^= v.x ^ v.y ^ v.z ^ v.w;
        }
    }
    if (acc == 0x9E3779B9u) sink[0] = acc;
}

}  // namespace

extern "C" {

// Reads `bytes` (a multiple of 16) from `buf` once; `sink` must hold one
// uint32 (`blocks` is accepted for compatibility and unused). Asynchronous on
// `stream`.
int mmbench_read(const void* buf, uint64_t bytes, void* sink, uint32_t blocks, void* stream) {
    (void)blocks;
    if (!buf || !sink || bytes % 16) return -2;
    const uint64_t n16 = bytes / 16;
    const uint64_t n_thr = (n16 + 3) / 4;
    const uint64_t grid = (n_thr + kThreads - 1) / kThreads;
    if (grid == 0 || grid > 0x7FFFFFFFu) return -2;
    read_kernel<<<(unsigned)grid, kThreads, 0, (hipStream_t)stream>>>((const u32x4*)buf, n16, n_thr,
                                                                     (uint32_t*)sink);
    return hipGetLastError() == hipSuccess ? 0 : -4;
}

}  // extern "C"
