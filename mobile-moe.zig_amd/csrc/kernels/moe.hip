// MoE routing and combine on gfx950 (moeFFN, inference.zig:886-1010).
//
// route_kernel: one workgroup, one wave per token. Each token runs
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

constexpr int kRouteThreads = 1024;  // 16 waves; one wave per token at a time
constexpr int kMaxTokens = 256;      // MMHIP_MOE_MAX_TOKENS
constexpr int kMaxExperts = 256;
constexpr int kMaxK = 4;

// The size-k min-heap of math.topK (math.zig:130-193) for k <= 4, held in
// registers: every position is a compile-time index, so siftDownMin's
// comparisons (children 2p+1, 2p+2 of parent p, strict <, left first) are
// spelled out for the only parents a heap of <= 4 entries has: 0 and 1.
struct Heap4 {
    uint32_t i0, i1, i2, i3;
    float s0, s1, s2, s3;
    __device__ void swap01() {
        uint32_t ti = i0; i0 = i1; i1 = ti;
        float ts = s0; s0 = s1; s1 = ts;
    }
    __device__ void swap02() {
        uint32_t ti = i0; i0 = i2; i2 = ti;
        float ts = s0; s0 = s2; s2 = ts;
    }
    __device__ void swap13() {
        uint32_t ti = i1; i1 = i3; i3 = ti;
        float ts = s1; s1 = s3; s3 = ts;
    }
    // siftDownMin(start = 1, end): the only child of position 1 is 3.
    __device__ void sift1(uint32_t end) {
        if (3 < end && s3 < s1) swap13();
    }
    // siftDownMin(start = 0, end).
    __device__ void sift0(uint32_t end) {
        uint32_t smallest = 0;
        float sm = s0;
        if (1 < end && s1 < sm) {
            smallest = 1;
            sm = s1;
        }
        if (2 < end && s2 < sm) smallest = 2;
        if (smallest == 1) {
            swap01();
            sift1(end);
        } else if (smallest == 2) {
            swap02();  // position 2 has no children below 4
        }
    }
};

// math.topK (math.zig:130-174): heap seeded with the first k scores, later
// scores replace the root only when strictly greater, results popped from the
// root into positions k-1, k-2, ... (descending). Run by a whole wave for one
// token: lane l holds scores l, l + 64, l + 128, l + 192 (n <= 256); the scan
// reads score j with readlane, so the heap's values are uniform registers.
__device__ float score_at(const float (&sc)[4], uint32_t j) {
    const float v = j < 64 ? sc[0] : j < 128 ? sc[1] : j < 192 ? sc[2] : sc[3];
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), (int)(j & 63)));
}

__device__ void top_k_wave(const float (&sc)[4], uint32_t n, uint32_t k, uint32_t (&ids)[kMaxK],
                           float (&ts)[kMaxK]) {
    Heap4 h;
    h.i0 = 0; h.s0 = score_at(sc, 0);
    h.i1 = 1; h.s1 = k > 1 ? score_at(sc, 1) : 0.0f;
    h.i2 = 2; h.s2 = k > 2 ? score_at(sc, 2) : 0.0f;
    h.i3 = 3; h.s3 = k > 3 ? score_at(sc, 3) : 0.0f;
    // for (i = k / 2; i > 0;) sift(--i, k)
    if (k / 2 >= 2) h.sift1(k);
    if (k / 2 >= 1) h.sift0(k);
    for (uint32_t j = k; j < n; ++j) {
        const float v = score_at(sc, j);
        if (v > h.s0) {
            h.i0 = j;
            h.s0 = v;
            h.sift0(k);
        }
    }
    // Pop: result[ri] = root; root = heap[ri]; sift(0, ri), ri = k-1 .. 0.
#pragma unroll
    for (int ri = kMaxK - 1; ri >= 0; --ri) {
        if ((uint32_t)ri >= k) continue;
        ids[ri] = h.i0;
        ts[ri] = h.s0;
        if (ri == 3) { h.i0 = h.i3; h.s0 = h.s3; }
        if (ri == 2) { h.i0 = h.i2; h.s0 = h.s2; }
        if (ri == 1) { h.i0 = h.i1; h.s0 = h.s1; }
        h.sift0((uint32_t)ri);
    }
}

// The common case of topK without the heap: when the k + 1 largest scores
// are distinct (and no score is NaN), the heap's result is exactly those k in
// descending order. k + 1 rounds of a wave-wide max find them; a repeated
// value in any round, or a NaN anywhere, returns false and the caller runs
// the heap (ties and NaNs make the heap's insertion order matter).
__device__ bool top_k_distinct(const float (&sc)[4], uint32_t n, uint32_t k, uint32_t (&ids)[kMaxK],
                               float (&ts)[kMaxK]) {
    const uint32_t lane = threadIdx.x & 63;
    uint32_t valid = 0;
    bool nan = false;
#pragma unroll
    for (int q = 0; q < 4; ++q)
        if (lane + 64 * q < n) {
            valid |= 1u << q;
            nan |= sc[q] != sc[q];
        }
    if (__any(nan)) return false;
    const uint32_t rounds = k < n ? k + 1 : k;
    for (uint32_t r = 0; r < rounds; ++r) {
        float best = -__builtin_inff();
        uint32_t best_q = 4, dup = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if (!((valid >> q) & 1u)) continue;
            if (best_q == 4 || sc[q] > best) {
                best = sc[q];
                best_q = q;
                dup = 0;
            } else if (sc[q] == best) {
                dup = 1;
            }
        }
        float m = best_q < 4 ? best : -__builtin_inff();
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
        const bool mine = best_q < 4 && best == m;
        const unsigned long long who = __ballot(mine);
        if (__popcll(who) != 1 || __any(mine && dup)) return false;
        const uint32_t wl = (uint32_t)__builtin_ctzll(who);
        const uint32_t wq = (uint32_t)__shfl((int)best_q, (int)wl, 64);
        if (r < k) {
            ids[r] = wl + 64 * wq;
            ts[r] = m;
        }
        if (lane == wl) valid &= ~(1u << wq);
    }
    return true;
}

__global__ __launch_bounds__(kRouteThreads) void route_kernel(RouteArgs a) {
    __shared__ uint32_t s_ids[kMaxTokens * kMaxK];
    __shared__ uint32_t s_act[kMaxTokens];  // bit i: assignment i of the token is computed
    __shared__ uint32_t s_cnt[kMaxExperts];   // assignments per expert
    __shared__ uint32_t s_off[kMaxExperts];   // first slot of each expert
    __shared__ uint32_t s_choff[kMaxExperts]; // first work item (chunk) of each expert
    __shared__ uint32_t s_rank[kMaxTokens * kMaxK];
    __shared__ uint32_t s_nchunks;
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63, wave = tid >> 6;
    const uint32_t T = a.n_tokens, E = a.n_experts, k = a.k;
    for (uint32_t e = tid; e < E; e += kRouteThreads) s_cnt[e] = 0;

    for (uint32_t t = wave; t < T; t += kRouteThreads / 64) {
        const BufRsrc sr = make_rsrc(a.scores + (uint64_t)t * E, E * 4);
        float sc[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) sc[q] = __uint_as_float(buf_load_b32(sr, (lane + 64 * q) * 4, 0));
        uint32_t ids[kMaxK] = {0, 0, 0, 0};
        float ts[kMaxK] = {0.f, 0.f, 0.f, 0.f}, w[kMaxK] = {0.f, 0.f, 0.f, 0.f};
        if (!top_k_distinct(sc, E, k, ids, ts)) top_k_wave(sc, E, k, ids, ts);
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
        // Heavy throttle keeps the top expert only and renormalises it
        // (225-242); the others are deferred.
        uint32_t act = (1u << k) - 1u, deferred = 0;
        if (a.level == 3 && k > 1) {
            act = 1u;
            deferred = 1;
            const float rem = 0.0f + w[0];
            if (rem > 0.0f) w[0] = w[0] * (a.scale / rem);
        }
        if (lane == 0) {
            for (uint32_t i = 0; i < k; ++i) atomicAdd(a.counts + ids[i], 1ull);  // stats.record (220-222)
            // RouteResult as moeFFN sees it (after the fallback).
            for (uint32_t i = 0; i < kMaxK; ++i) {
                if (a.route_ids) a.route_ids[t * kMaxK + i] = i < k ? ids[i] : 0xFFFFFFFFu;
                if (a.route_w) a.route_w[t * kMaxK + i] = i < k ? w[i] : 0.0f;
                s_ids[t * kMaxK + i] = ids[i];
                a.assign_w[t * kMaxK + i] = ((act >> i) & 1u) ? w[i] : 0.0f;
                a.assign_slot[t * kMaxK + i] = -1;
            }
            s_act[t] = act;
            a.deferred[t] = deferred;
            a.shared_slot[t] = a.shared ? (int32_t)(4 * T + t) : -1;
            a.slot_tok[4 * T + t] = t;
        }
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

    // Prefill: assignments grouped by expert. An assignment's rank inside its
    // expert group comes from an LDS counter; rows of a group are independent,
    // so the order inside a group does not change any result.
    for (uint32_t p = tid; p < T * kMaxK; p += kRouteThreads) {
        const uint32_t t = p / kMaxK, i = p % kMaxK;
        if (i < k && ((s_act[t] >> i) & 1u)) s_rank[p] = atomicAdd(&s_cnt[s_ids[p]], 1u);
    }
    __syncthreads();
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
        if (lane == 0) s_nchunks = carry_ch;
    }
    __syncthreads();
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
    const uint32_t nch = s_nchunks;
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
    if (a.n_tokens == 0 || a.n_tokens > kMaxTokens || a.n_experts > kMaxExperts || a.k == 0 || a.k > kMaxK ||
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
