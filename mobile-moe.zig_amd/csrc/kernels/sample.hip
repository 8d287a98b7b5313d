// Greedy sampling on gfx950: sampleGreedy (inference.zig:376-386) over the
// logits that computeLogits (inference.zig:1189-1197) produces with the
// output projection GEMV (gemv.hip / gemv_iq2.hip).
//
// Two launches: workgroups of 256 threads each take 2,048 consecutive logits
// and write the first index of their largest value (a partial), then one
// workgroup combines the partials. Each thread scans its values in ascending
// index order (four consecutive per step, both steps' loads in flight),
// keeping the first of equal maxima with a strict >; waves and workgroups
// combine (value, index) pairs, a larger value or an equal value at a
// smaller index winning. NaN values never enter; a NaN logits[0] gives 0, as
// the sequential scan, whose first candidate is logits[0], never displaces it.
#include "device_common.hpp"
#include "kernels.hpp"

namespace mmhip {

namespace {

constexpr int kArgThreads = 256;
constexpr uint32_t kArgChunk = 2048;  // logits per first-pass workgroup
constexpr uint32_t kArgNone = 0xFFFFFFFFu;

__device__ __forceinline__ void take_better(float& v, uint32_t& i, float v2, uint32_t i2) {
    if (i2 != kArgNone && (i == kArgNone || v2 > v || (v2 == v && i2 < i))) {
        v = v2;
        i = i2;
    }
}

// The workgroup's best pair (valid in thread 0).
__device__ __forceinline__ void reduce_pairs(float& bv, uint32_t& bi) {
    __shared__ float sv[kArgThreads / 64];
    __shared__ uint32_t si[kArgThreads / 64];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float v2 = __shfl_xor(bv, off, 64);
        const uint32_t i2 = (uint32_t)__shfl_xor((int)bi, off, 64);
        take_better(bv, bi, v2, i2);
    }
    if ((threadIdx.x & 63) == 0) {
        sv[threadIdx.x >> 6] = bv;
        si[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
#pragma unroll
        for (int w = 1; w < kArgThreads / 64; ++w) take_better(bv, bi, sv[w], si[w]);
    }
}

__global__ __launch_bounds__(kArgThreads) void argmax_partial_kernel(const float* __restrict__ x, uint32_t n,
                                                                     float* __restrict__ pv,
                                                                     uint32_t* __restrict__ pi) {
    const bool vec = (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
    const uint32_t c0 = blockIdx.x * kArgChunk;
    float v[kArgChunk / kArgThreads];
#pragma unroll
    for (uint32_t s = 0; s < kArgChunk / (kArgThreads * 4); ++s) {
        const uint32_t base = c0 + (s * kArgThreads + threadIdx.x) * 4;
        if (vec && base + 4 <= n) {
            const float4 q = *reinterpret_cast<const float4*>(x + base);
            v[4 * s] = q.x;
            v[4 * s + 1] = q.y;
            v[4 * s + 2] = q.z;
            v[4 * s + 3] = q.w;
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[4 * s + e] = base + e < n ? x[base + e] : __builtin_nanf("");
        }
    }
    float bv = 0.0f;
    uint32_t bi = kArgNone;
#pragma unroll
    for (uint32_t s = 0; s < kArgChunk / (kArgThreads * 4); ++s)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float w = v[4 * s + e];
            if (w == w && (bi == kArgNone || w > bv)) {
                bv = w;
                bi = c0 + (s * kArgThreads + threadIdx.x) * 4 + e;
            }
        }
    reduce_pairs(bv, bi);
    if (threadIdx.x == 0) {
        pv[blockIdx.x] = bv;
        pi[blockIdx.x] = bi;
    }
}

__global__ __launch_bounds__(kArgThreads) void argmax_final_kernel(const float* __restrict__ x,
                                                                   const float* __restrict__ pv,
                                                                   const uint32_t* __restrict__ pi, uint32_t g,
                                                                   uint32_t* __restrict__ out) {
    float bv = 0.0f;
    uint32_t bi = kArgNone;
    for (uint32_t b = threadIdx.x; b < g; b += kArgThreads) take_better(bv, bi, pv[b], pi[b]);
    reduce_pairs(bv, bi);
    if (threadIdx.x == 0) {
        const float x0 = x[0];
        *out = (x0 != x0 || bi == kArgNone) ? 0u : bi;
    }
}

}  // namespace

uint64_t argmax_scratch_bytes(uint64_t n) { return (n + kArgChunk - 1) / kArgChunk * 8; }

hipError_t launch_argmax(const float* x, uint64_t n, uint32_t* out, void* scratch, hipStream_t s) {
    if (n == 0 || n > 0xFFFFFFFFull || !scratch) return hipErrorInvalidValue;
    const uint32_t g = (uint32_t)((n + kArgChunk - 1) / kArgChunk);
    float* pv = static_cast<float*>(scratch);
    uint32_t* pi = reinterpret_cast<uint32_t*>(pv + g);
    argmax_partial_kernel<<<g, kArgThreads, 0, s>>>(x, (uint32_t)n, pv, pi);
    argmax_final_kernel<<<1, kArgThreads, 0, s>>>(x, pv, pi, g, out);
    return hipGetLastError();
}

}  // namespace mmhip
