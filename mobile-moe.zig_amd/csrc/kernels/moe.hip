// MoE routing and combine on gfx950 (moeFFN, inference.zig:886-1010).
//
// route_kernel: one workgroup, one thread per token. Each token runs
// Scheduler.route exactly as the CPU path does (math.topK's size-k min-heap,
// softmax over the selected logits, throttle scaling, the heavy-throttle
// top-1 fallback) and counts its experts (ExpertStats.counts). The workgroup
// then lays out the activation slots of the call and writes the problem
// lists that the expert kernels read on the device, so no routing result
// travels back to the host:
//   n_tokens == 1: GEMV problems in route order (decode);
//   n_tokens >  1: assignments sorted by expert (tokens in order) and cut
//                  into QMM work items of <= kQmmTokens rows (prefill).
// combine_kernel: the weighted sum in route order, the shared expert and the
// deferral bias, with products and sums rounded separately as on the CPU.
#include "device_common.hpp"
#include "kernels.hpp"

namespace mmhip {

namespace {

constexpr int kRouteThreads = 256;  // >= MMHIP_MOE_MAX_TOKENS
constexpr int kMaxK = 4;

// math.siftDownMin (math.zig:177-193).
__device__ void sift_down_min(uint32_t (&hi)[kMaxK], float (&hs)[kMaxK], uint32_t start, uint32_t end) {
    uint32_t parent = start;
    for (;;) {
        const uint32_t left = parent * 2 + 1, right = left + 1;
        uint32_t smallest = parent;
        if (left < end && hs[left] < hs[smallest]) smallest = left;
        if (right < end && hs[right] < hs[smallest]) smallest = right;
        if (smallest == parent) break;
        const uint32_t ti = hi[parent];
        hi[parent] = hi[smallest];
        hi[smallest] = ti;
        const float ts = hs[parent];
        hs[parent] = hs[smallest];
        hs[smallest] = ts;
        parent = smallest;
    }
}

// math.topK (math.zig:130-174): heap seeded with the first k scores, later
// scores replace the root only when strictly greater, results popped from the
// root into positions k-1, k-2, ... (descending).
__device__ void top_k(const float* scores, uint32_t n, uint32_t k, uint32_t (&ids)[kMaxK], float (&ts)[kMaxK]) {
    uint32_t hi[kMaxK];
    float hs[kMaxK];
    for (uint32_t i = 0; i < k; ++i) {
        hi[i] = i;
        hs[i] = scores[i];
    }
    for (uint32_t i = k / 2; i > 0;) {
        --i;
        sift_down_min(hi, hs, i, k);
    }
    for (uint32_t j = k; j < n; ++j) {
        const float v = scores[j];
        if (v > hs[0]) {
            hi[0] = j;
            hs[0] = v;
            sift_down_min(hi, hs, 0, k);
        }
    }
    for (uint32_t ri = k; ri > 0;) {
        --ri;
        ids[ri] = hi[0];
        ts[ri] = hs[0];
        hi[0] = hi[ri];
        hs[0] = hs[ri];
        sift_down_min(hi, hs, 0, ri);
    }
}

__global__ __launch_bounds__(kRouteThreads) void route_kernel(RouteArgs a) {
    __shared__ uint32_t s_ids[kRouteThreads * kMaxK];
    __shared__ uint32_t s_act[kRouteThreads];  // bit i: assignment i of the token is computed
    __shared__ uint32_t s_cnt[kRouteThreads];  // per expert (n_experts <= kRouteThreads)
    __shared__ uint32_t s_off[kRouteThreads];
    const uint32_t tid = threadIdx.x;
    const uint32_t T = a.n_tokens, E = a.n_experts, k = a.k;

    if (tid < T) {
        const uint32_t t = tid;
        uint32_t ids[kMaxK] = {0, 0, 0, 0};
        float ts[kMaxK] = {0.f, 0.f, 0.f, 0.f}, w[kMaxK] = {0.f, 0.f, 0.f, 0.f};
        top_k(a.scores + (uint64_t)t * E, E, k, ids, ts);
        // Softmax over the selected logits, then the routed scaling factor
        // (scheduler.zig:184-201).
        float mx = ts[0];
        for (uint32_t i = 1; i < k; ++i)
            if (ts[i] > mx) mx = ts[i];
        float sum = 0.0f;
        for (uint32_t i = 0; i < k; ++i) {
            w[i] = expf(ts[i] - mx);
            sum = sum + w[i];
        }
        for (uint32_t i = 0; i < k; ++i) w[i] = w[i] / sum;
        for (uint32_t i = 0; i < k; ++i) w[i] = w[i] * a.scale;
        for (uint32_t i = 0; i < k; ++i) atomicAdd(a.counts + ids[i], 1ull);  // stats.record (220-222)
        // Heavy throttle keeps the top expert only and renormalises it
        // (225-242); the others are deferred.
        uint32_t act = (1u << k) - 1u, deferred = 0;
        if (a.level == 3 && k > 1) {
            act = 1u;
            deferred = 1;
            const float rem = 0.0f + w[0];
            if (rem > 0.0f) w[0] = w[0] * (a.scale / rem);
        }
        // RouteResult as moeFFN sees it (after the fallback).
        if (a.route_ids)
            for (uint32_t i = 0; i < kMaxK; ++i) a.route_ids[t * kMaxK + i] = i < k ? ids[i] : 0xFFFFFFFFu;
        if (a.route_w)
            for (uint32_t i = 0; i < kMaxK; ++i) a.route_w[t * kMaxK + i] = i < k ? w[i] : 0.0f;
        for (uint32_t i = 0; i < kMaxK; ++i) {
            s_ids[t * kMaxK + i] = ids[i];
            a.assign_w[t * kMaxK + i] = ((act >> i) & 1u) ? w[i] : 0.0f;
            a.assign_slot[t * kMaxK + i] = -1;
        }
        s_act[t] = act;
        a.deferred[t] = deferred;
        a.shared_slot[t] = a.shared ? (int32_t)(4 * T + t) : -1;
        a.slot_tok[4 * T + t] = t;
    }
    __syncthreads();

    if (T == 1) {
        // Decode: slots in route order; GEMV problem lists.
        if (tid == 0) {
            uint32_t s = 0;
            for (uint32_t i = 0; i < k; ++i) {
                if (!((s_act[0] >> i) & 1u)) continue;
                const uint32_t e = s_ids[i];
                a.assign_slot[i] = (int32_t)s;
                a.slot_tok[s] = 0;
                a.gemv_gu[2 * s] = make_uint4(e, 0, 2 * s, 0);
                a.gemv_gu[2 * s + 1] = make_uint4(E + e, 0, 2 * s + 1, 0);
                a.gemv_dn[s] = make_uint4(e, s, s, 0);
                ++s;
            }
            uint32_t n_gu = 2 * s, n_dn = s;
            if (a.shared && a.shared_merged) {
                a.gemv_gu[n_gu++] = make_uint4(2 * E, 0, 8, 0);
                a.gemv_gu[n_gu++] = make_uint4(2 * E + 1, 0, 9, 0);
                a.gemv_dn[n_dn++] = make_uint4(E, 4, 4, 0);
            }
            a.n_gemv[0] = n_gu;
            a.n_gemv[1] = n_dn;
        }
        return;
    }

    // Prefill: assignments sorted by expert, tokens in order within an expert.
    for (uint32_t e = tid; e < E; e += kRouteThreads) {
        uint32_t c = 0;
        for (uint32_t t = 0; t < T; ++t)
            for (uint32_t i = 0; i < k; ++i) c += (((s_act[t] >> i) & 1u) && s_ids[t * kMaxK + i] == e) ? 1u : 0u;
        s_cnt[e] = c;
    }
    __syncthreads();
    if (tid == 0) {
        uint32_t off = 0;
        for (uint32_t e = 0; e < E; ++e) {
            s_off[e] = off;
            off += s_cnt[e];
        }
    }
    __syncthreads();
    for (uint32_t e = tid; e < E; e += kRouteThreads) {
        uint32_t r = s_off[e];
        for (uint32_t t = 0; t < T; ++t)
            for (uint32_t i = 0; i < k; ++i)
                if (((s_act[t] >> i) & 1u) && s_ids[t * kMaxK + i] == e) {
                    a.assign_slot[t * kMaxK + i] = (int32_t)r;
                    a.slot_tok[r] = t;
                    ++r;
                }
    }
    if (tid == 0) {
        uint32_t ng = 0, nd = 0;
        for (uint32_t e = 0; e < E; ++e) {
            const uint32_t c = s_cnt[e], off = s_off[e];
            for (uint32_t c0 = 0; c0 < c; c0 += kQmmTokens) {
                const uint32_t m = min(kQmmTokens, c - c0);
                a.work_gu[ng++] = QmmWork{e, off + c0, m, 0};
                a.work_gu[ng++] = QmmWork{E + e, off + c0, m, a.inter};
                a.work_dn[nd++] = QmmWork{e, off + c0, m, 0};
            }
        }
        if (a.shared && a.shared_merged) {
            for (uint32_t c0 = 0; c0 < T; c0 += kQmmTokens) {
                const uint32_t m = min(kQmmTokens, T - c0);
                a.work_gu[ng++] = QmmWork{2 * E, 4 * T + c0, m, 0};
                a.work_gu[ng++] = QmmWork{2 * E + 1, 4 * T + c0, m, a.inter};
                a.work_dn[nd++] = QmmWork{E, 4 * T + c0, m, 0};
            }
        }
        a.n_work[0] = ng;
        a.n_work[1] = nd;
    }
}

__global__ void combine_kernel(const float* __restrict__ eo, const int32_t* __restrict__ assign_slot,
                               const float* __restrict__ assign_w, const int32_t* __restrict__ shared_slot,
                               const uint32_t* __restrict__ deferred, const float* __restrict__ bias,
                               float* __restrict__ out, uint32_t n_tokens, uint32_t hidden) {
    const uint64_t gid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= (uint64_t)n_tokens * hidden) return;
    const uint32_t t = (uint32_t)(gid / hidden), j = (uint32_t)(gid % hidden);
    float o = 0.0f;
#pragma unroll
    for (int i = 0; i < kMaxK; ++i) {
        const int32_t s = assign_slot[t * kMaxK + i];
        if (s >= 0) o = __fadd_rn(o, __fmul_rn(assign_w[t * kMaxK + i], eo[(uint64_t)s * hidden + j]));
    }
    const int32_t sh = shared_slot[t];
    if (sh >= 0) o = __fadd_rn(o, eo[(uint64_t)sh * hidden + j]);
    if (bias && deferred[t]) o = __fadd_rn(o, bias[j]);
    out[gid] = o;
}

}  // namespace

uint32_t route_max_work(uint32_t n_tokens, uint32_t n_experts) {
    const uint32_t routed = 4 * n_tokens;
    const uint32_t chunks = (n_experts < routed ? n_experts : routed) + (routed + kQmmTokens - 1) / kQmmTokens +
                            (n_tokens + kQmmTokens - 1) / kQmmTokens;
    return 2 * chunks;
}

hipError_t launch_route(const RouteArgs& a, hipStream_t s) {
    if (a.n_tokens == 0 || a.n_tokens > kRouteThreads || a.n_experts > kRouteThreads || a.k == 0 || a.k > kMaxK ||
        a.k > a.n_experts)
        return hipErrorInvalidValue;
    route_kernel<<<1, kRouteThreads, 0, s>>>(a);
    return hipGetLastError();
}

hipError_t launch_combine(const float* eo, const int32_t* assign_slot, const float* assign_w,
                          const int32_t* shared_slot, const uint32_t* deferred, const float* bias, float* out,
                          uint32_t n_tokens, uint32_t hidden, hipStream_t s) {
    const uint64_t n = (uint64_t)n_tokens * hidden;
    if (n == 0) return hipSuccess;
    combine_kernel<<<(unsigned)((n + 255) / 256), 256, 0, s>>>(eo, assign_slot, assign_w, shared_slot, deferred, bias,
                                                               out, n_tokens, hidden);
    return hipGetLastError();
}

}  // namespace mmhip
