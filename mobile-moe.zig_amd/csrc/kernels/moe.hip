// MoE routing and combine on gfx950 (moeFFN, inference.zig:886-1010).
//
// route_kernel: workgroup 0 routes, four tokens per wave (one per 16-lane
// row); any further workgroups quantise the hidden states for the grouped
// gate/up meanwhile (one wave per token and 256-column unit). Each token runs
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
#include "route_ops.hpp"

namespace mmhip {

namespace {

constexpr int kRouteThreads = 1024;  // 16 waves, 4 tokens each at a time
constexpr int kMaxTokens = 256;      // MMHIP_MOE_MAX_TOKENS
constexpr int kMaxExperts = 256;

// LDS of the routing pass (one workgroup of kRouteThreads threads).
struct RouteLds {
    uint32_t ids[kMaxTokens * kMaxK];
    uint32_t act[kMaxTokens];    // bit i: assignment i of the token is computed
    uint32_t cnt[kMaxExperts];   // assignments per expert
    uint32_t rec[kMaxExperts];   // experts recorded in the statistics this call
    uint32_t off[kMaxExperts];   // first slot of each expert
    uint32_t choff[kMaxExperts]; // first work item (chunk) of each expert
    uint32_t rank[kMaxTokens * kMaxK];
    uint32_t nchunks;
};

__device__ void route_body(const RouteArgs& a, RouteLds& L) {
    uint32_t* const s_ids = L.ids;
    uint32_t* const s_act = L.act;
    uint32_t* const s_cnt = L.cnt;
    uint32_t* const s_rec = L.rec;
    uint32_t* const s_off = L.off;
    uint32_t* const s_choff = L.choff;
    uint32_t* const s_rank = L.rank;
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t T = a.n_tokens, E = a.n_experts, k = a.k;
    for (uint32_t e = tid; e < E; e += kRouteThreads) {
        s_cnt[e] = 0;
        s_rec[e] = 0;
    }
    // Every barrier here orders LDS only: no phase reads what an earlier one
    // stored to global memory, and __syncthreads() would also wait for every
    // wave's outstanding global stores and statistics atomics (~1 us each).
    lds_barrier();

    // Four tokens per wave, one per 16-lane row (route_row16); the row's
    // first lane writes the token's results.
    for (uint32_t t0 = 4 * wave; t0 < T; t0 += 4 * (kRouteThreads / 64)) {
        const uint32_t t = t0 + (lane >> 4);
        const TokenRoute tr = E <= 64 ? route_row16<4>(a, t) : route_row16<16>(a, t);
        if ((lane & 15) == 0 && t < T) {
            const uint32_t act = tr.act;
#pragma unroll
            for (uint32_t i = 0; i < kMaxK; ++i)
                if (i < k) atomicAdd(&s_rec[tr.ids[i]], 1u);  // stats.record (220-222)
            // RouteResult as moeFFN sees it (after the fallback).
#pragma unroll
            for (uint32_t i = 0; i < kMaxK; ++i) {
                if (a.route_ids) a.route_ids[t * kMaxK + i] = i < k ? tr.ids[i] : 0xFFFFFFFFu;
                if (a.route_w) a.route_w[t * kMaxK + i] = i < k ? tr.w[i] : 0.0f;
                s_ids[t * kMaxK + i] = tr.ids[i];
                a.assign_w[t * kMaxK + i] = ((act >> i) & 1u) ? tr.w[i] : 0.0f;
                a.assign_slot[t * kMaxK + i] = -1;
            }
            s_act[t] = act;
            a.deferred[t] = tr.deferred;
            a.shared_slot[t] = a.shared ? (int32_t)(4 * T + t) : -1;
            a.slot_tok[4 * T + t] = t;
        }
    }
    lds_barrier();
    // Statistics: one device atomic per recorded expert.
    for (uint32_t e = tid; e < E; e += kRouteThreads)
        if (s_rec[e]) atomicAdd(a.counts + e, (unsigned long long)s_rec[e]);

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

    // Prefill: assignments grouped by expert. An assignment's rank inside its
    // expert group comes from an LDS counter; rows of a group are independent,
    // so the order inside a group does not change any result.
    for (uint32_t p = tid; p < T * kMaxK; p += kRouteThreads) {
        const uint32_t t = p / kMaxK, i = p % kMaxK;
        if (i < k && ((s_act[t] >> i) & 1u)) s_rank[p] = atomicAdd(&s_cnt[s_ids[p]], 1u);
    }
    lds_barrier();
    if (wave == 0) {
        // Exclusive scans over experts: slot offsets and chunk (work item) offsets.
        uint32_t carry = 0, carry_ch = 0;
        for (uint32_t base = 0; base < E; base += 64) {
            const uint32_t e = base + lane;
            const uint32_t c = e < E ? s_cnt[e] : 0u;
            const uint32_t ch = (c + kQmmTokens - 1) / kQmmTokens;
            uint32_t inc = c, inc_ch = ch;
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const uint32_t u = (uint32_t)__shfl_up((int)inc, off, 64);
                const uint32_t uch = (uint32_t)__shfl_up((int)inc_ch, off, 64);
                if (lane >= (uint32_t)off) {
                    inc += u;
                    inc_ch += uch;
                }
            }
            if (e < E) {
                s_off[e] = carry + inc - c;
                s_choff[e] = carry_ch + inc_ch - ch;
            }
            carry += (uint32_t)__shfl((int)inc, 63, 64);
            carry_ch += (uint32_t)__shfl((int)inc_ch, 63, 64);
        }
        if (lane == 0) L.nchunks = carry_ch;
    }
    lds_barrier();
    for (uint32_t p = tid; p < T * kMaxK; p += kRouteThreads) {
        const uint32_t t = p / kMaxK, i = p % kMaxK;
        if (i < k && ((s_act[t] >> i) & 1u)) {
            const uint32_t slot = s_off[s_ids[p]] + s_rank[p];
            a.assign_slot[p] = (int32_t)slot;
            a.slot_tok[slot] = t;
        }
    }
    // Work items: chunk c of expert e is item s_choff[e] + c (gate and up
    // interleaved in the gate/up list); the shared expert's chunks follow.
    for (uint32_t e = tid; e < E; e += kRouteThreads) {
        const uint32_t c = s_cnt[e], off = s_off[e], ch0 = s_choff[e];
        for (uint32_t c0 = 0, q = ch0; c0 < c; c0 += kQmmTokens, ++q) {
            const uint32_t m = min(kQmmTokens, c - c0);
            a.work_gu[2 * q] = QmmWork{e, off + c0, m, 0};
            a.work_gu[2 * q + 1] = QmmWork{E + e, off + c0, m, a.inter};
            a.work_dn[q] = QmmWork{e, off + c0, m, 0};
        }
    }
    const uint32_t nch = L.nchunks;
    const bool sh = a.shared && a.shared_merged;
    const uint32_t sh_chunks = sh ? (T + kQmmTokens - 1) / kQmmTokens : 0;
    for (uint32_t c = tid; c < sh_chunks; c += kRouteThreads) {
        const uint32_t c0 = c * kQmmTokens, m = min(kQmmTokens, T - c0), q = nch + c;
        a.work_gu[2 * q] = QmmWork{2 * E, 4 * T + c0, m, 0};
        a.work_gu[2 * q + 1] = QmmWork{2 * E + 1, 4 * T + c0, m, a.inter};
        a.work_dn[q] = QmmWork{E, 4 * T + c0, m, 0};
    }
    if (tid == 0) {
        a.n_work[0] = 2 * (nch + sh_chunks);
        a.n_work[1] = nch + sh_chunks;
    }
}

__global__ __launch_bounds__(kRouteThreads) void route_kernel(RouteArgs a) {
    __shared__ RouteLds L;
    if (blockIdx.x > 0) {
        // Hidden-state quantisation: one wave per (token, 256-column unit).
        const uint64_t unit = (uint64_t)(blockIdx.x - 1) * (kRouteThreads / 64) + (threadIdx.x >> 6);
        if (unit < (uint64_t)a.n_tokens * a.q_units)
            quantize_unit_wave<false>(a.qx, a.qx_stride, 0, unit / a.q_units, (uint32_t)(unit % a.q_units), a.q_cols,
                                      a.qa.hi, a.qa.lo, a.qa.scale, a.qa.stride, a.qa.scale_stride);
        return;
    }
    route_body(a, L);
}


__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ eo, const int32_t* __restrict__ assign_slot,
                               const float* __restrict__ assign_w, const int32_t* __restrict__ shared_slot,
                               const uint32_t* __restrict__ deferred, const float* __restrict__ bias,
                               float* __restrict__ out, uint32_t n_tokens, uint32_t hidden) {
    // All arguments in one batch of scalar loads (the bounds check below
    // otherwise waited for its own first: one more round trip).
    asm volatile("" ::"s"(eo), "s"(assign_slot), "s"(assign_w), "s"(shared_slot), "s"(deferred), "s"(bias), "s"(out),
                 "s"(n_tokens), "s"(hidden));
    const uint64_t gid = (uint64_t)blockIdx.x * 256 + threadIdx.x;  // 256 threads (launch_combine)
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
    if (a.n_tokens == 0 || a.n_tokens > kMaxTokens || a.n_experts > kMaxExperts || a.k == 0 || a.k > kMaxK ||
        a.k > a.n_experts)
        return hipErrorInvalidValue;
    const uint64_t q_waves = a.qx ? (uint64_t)a.n_tokens * a.q_units : 0;
    const unsigned q_wgs = (unsigned)((q_waves + kRouteThreads / 64 - 1) / (kRouteThreads / 64));
    route_kernel<<<1 + q_wgs, kRouteThreads, 0, s>>>(a);
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
