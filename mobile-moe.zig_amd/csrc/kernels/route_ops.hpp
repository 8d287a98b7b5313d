// Routing of one token (Scheduler.route, scheduler.zig:169-262), run by a
// whole wave: math.topK over the router scores, softmax over the selected
// logits, the routed scaling factor and the heavy-throttle top-1 fallback.
// Shared by the routing kernel and the decode gate/up GEMV, which routes
// its single token itself (every wave computes the same result).
#pragma once

#include "device_common.hpp"
#include "kernels.hpp"

namespace mmhip {

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
__device__ __forceinline__ float score_at(const float (&sc)[4], uint32_t j) {
    // Uniform branches, one readlane each: a select over the four registers
    // would be lowered to an indexed scratch access.
    const int l = (int)(j & 63u);
    const uint32_t q = j >> 6;
    if (q == 0) return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sc[0]), l));
    if (q == 1) return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sc[1]), l));
    if (q == 2) return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sc[2]), l));
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sc[3]), l));
}

// math.topK (math.zig:130-174) over scores get(0 .. n-1).
template <typename Get>
__device__ inline void top_k_heap(Get get, uint32_t n, uint32_t k, uint32_t (&ids)[kMaxK], float (&ts)[kMaxK]) {
    Heap4 h;
    h.i0 = 0; h.s0 = get(0);
    h.i1 = 1; h.s1 = k > 1 ? get(1) : 0.0f;
    h.i2 = 2; h.s2 = k > 2 ? get(2) : 0.0f;
    h.i3 = 3; h.s3 = k > 3 ? get(3) : 0.0f;
    // for (i = k / 2; i > 0;) sift(--i, k)
    if (k / 2 >= 2) h.sift1(k);
    if (k / 2 >= 1) h.sift0(k);
    for (uint32_t j = k; j < n; ++j) {
        const float v = get(j);
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

// One token per wave: the scores live one per lane (score_at).
__device__ inline void top_k_wave(const float (&sc)[4], uint32_t n, uint32_t k, uint32_t (&ids)[kMaxK],
                                  float (&ts)[kMaxK]) {
    top_k_heap([&](uint32_t j) { return score_at(sc, j); }, n, k, ids, ts);
}

// The common case of topK without the heap: when the k + 1 largest scores
// are distinct (and no score is NaN), the heap's result is exactly those k in
// descending order. k + 1 rounds of a wave-wide max find them; a repeated
// value in any round, or a NaN anywhere, returns false and the caller runs
// the heap (ties and NaNs make the heap's insertion order matter).
__device__ inline bool top_k_distinct(const float (&sc)[4], uint32_t n, uint32_t k, uint32_t (&ids)[kMaxK],
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
#pragma unroll
    for (uint32_t r = 0; r < kMaxK + 1; ++r) {  // constant r: ids / ts stay in registers
        if (r >= rounds) break;
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
        const float m = wave_max(best_q < 4 ? best : -__builtin_inff());
        const bool mine = best_q < 4 && best == m;
        const unsigned long long who = __ballot(mine);
        if (__popcll(who) != 1 || __any(mine && dup)) return false;
        const uint32_t wl = (uint32_t)__builtin_ctzll(who);
        const uint32_t wq = (uint32_t)__builtin_amdgcn_readlane((int)best_q, (int)wl);
        if (r < k) {
            ids[r] = wl + 64 * wq;
            ts[r] = m;
        }
        if (lane == wl) valid &= ~(1u << wq);
    }
    return true;
}

// The routing of token t (uniform across the wave). ids / w hold the k
// selected experts in topK order and their weights after the fallback; bit i
// of act is set when assignment i is computed; deferred is the fallback flag.
struct TokenRoute {
    uint32_t ids[kMaxK];
    float w[kMaxK];
    uint32_t act, deferred;
};
// Router scores of token t, lane l holding experts l, l + 64, l + 128, l + 192
// (experts past n_experts read as zero and are never selected).
__device__ inline void load_scores(const RouteArgs& a, uint32_t t, float (&sc)[4]) {
    const uint32_t lane = threadIdx.x & 63;
    const BufRsrc sr = make_rsrc(a.scores + (uint64_t)t * a.n_experts, a.n_experts * 4);
#pragma unroll
    for (int q = 0; q < 4; ++q) sc[q] = __uint_as_float(buf_load_b32(sr, (lane + 64 * q) * 4, 0));
}

// Which of the k selected experts are computed (bit i: assignment i) and
// whether the others are deferred: all of them, except under the heavy
// throttle, which keeps the top expert only (scheduler.zig:225-242). Known
// from the ids alone, before the weights.
__device__ __forceinline__ void route_active(const RouteArgs& a, uint32_t& act, uint32_t& deferred) {
    const bool heavy = a.level == 3 && a.k > 1;
    act = heavy ? 1u : (1u << a.k) - 1u;
    deferred = heavy ? 1u : 0u;
}

// Route weights of the selected experts (ids, logits ts in topK order).
__device__ inline TokenRoute finish_route(const RouteArgs& a, const uint32_t (&ids)[kMaxK], const float (&ts)[kMaxK]) {
    const uint32_t k = a.k;
    TokenRoute r{{ids[0], ids[1], ids[2], ids[3]}, {0.f, 0.f, 0.f, 0.f}, 0, 0};
    // Softmax over the selected logits, then the routed scaling factor
    // (scheduler.zig:184-201). Loops run over kMaxK with a k test so that
    // every array index is a compile-time constant (registers, no scratch).
    float mx = ts[0];
#pragma unroll
    for (uint32_t i = 1; i < kMaxK; ++i)
        if (i < k && ts[i] > mx) mx = ts[i];
    float sum = 0.0f;
#pragma unroll
    for (uint32_t i = 0; i < kMaxK; ++i)
        if (i < k) {
            r.w[i] = expf(ts[i] - mx);
            sum = sum + r.w[i];
        }
#pragma unroll
    for (uint32_t i = 0; i < kMaxK; ++i)
        if (i < k) r.w[i] = r.w[i] / sum;
#pragma unroll
    for (uint32_t i = 0; i < kMaxK; ++i)
        if (i < k) r.w[i] = r.w[i] * a.scale;
    // Heavy throttle keeps the top expert only and renormalises it
    // (225-242); the others are deferred.
    route_active(a, r.act, r.deferred);
    if (r.deferred) {
        const float rem = 0.0f + r.w[0];
        if (rem > 0.0f) r.w[0] = r.w[0] * (a.scale / rem);
    }
    return r;
}

// Integer key of a float whose signed order is the float order (NaN aside):
// negative values get their magnitude bits flipped. -0 and +0 get different
// keys; callers detect equal floats by a float compare.
__device__ __forceinline__ int order_key(float f) {
    const int b = __float_as_int(f);
    return b ^ ((b >> 31) & 0x7FFFFFFF);
}
__device__ __forceinline__ float key_float(int k) { return __int_as_float(k ^ ((k >> 31) & 0x7FFFFFFF)); }

// Wave-wide signed max, every lane receives it (the DPP steps of wave_max on
// integers: no float canonicalisation between steps).
__device__ __forceinline__ int wave_max_i32(int v) {
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false));
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false));
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false));
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false));
    const auto p = __builtin_amdgcn_permlane16_swap((uint32_t)v, (uint32_t)v, false, false);
    v = max((int)p[0], (int)p[1]);
    const auto q = __builtin_amdgcn_permlane32_swap((uint32_t)v, (uint32_t)v, false, false);
    return max((int)q[0], (int)q[1]);
}

// top_k_distinct for n <= 64 (score j in lane j): each of the k rounds
// takes the largest remaining key and fails (heap fallback) unless exactly
// one remaining score equals it as a float (which also catches -0 against
// +0). When all k rounds succeed, the k picks are distinct and strictly
// above every other score, so math.topK returns them in this order whatever
// its insertion order. No live key is kKeyNone: only a NaN maps there.
constexpr int kKeyNone = (int)0x80000000;
__device__ inline bool top_k_distinct64(float v, uint32_t n, uint32_t k, uint32_t (&ids)[kMaxK],
                                        float (&ts)[kMaxK]) {
    const uint32_t lane = threadIdx.x & 63;
    bool live = lane < n;
    if (__any(live && v != v)) return false;
    int key = live ? order_key(v) : kKeyNone;
#pragma unroll
    for (uint32_t r = 0; r < kMaxK; ++r) {  // constant r: ids / ts stay in registers
        if (r >= k) break;
        const float m = key_float(wave_max_i32(key));
        const unsigned long long who = __ballot(live && v == m);
        if (__popcll(who) != 1) return false;
        const uint32_t wl = (uint32_t)__builtin_ctzll(who);
        ids[r] = wl;
        ts[r] = m;
        if (lane == wl) {
            live = false;
            key = kKeyNone;
        }
    }
    return true;
}

// The k selected experts of one token and their logits in topK order, by a
// whole wave (scores one per lane).
__device__ inline void route_select(const RouteArgs& a, const float (&sc)[4], uint32_t (&ids)[kMaxK],
                                    float (&ts)[kMaxK]) {
#pragma unroll
    for (uint32_t i = 0; i < kMaxK; ++i) {
        ids[i] = 0;
        ts[i] = 0.0f;
    }
    const bool fast = a.n_experts <= 64 ? top_k_distinct64(sc[0], a.n_experts, a.k, ids, ts)
                                        : top_k_distinct(sc, a.n_experts, a.k, ids, ts);
    if (!fast) top_k_wave(sc, a.n_experts, a.k, ids, ts);
}

// Routing of one token by a whole wave (scores one per lane).
__device__ inline TokenRoute route_scores(const RouteArgs& a, const float (&sc)[4]) {
    uint32_t ids[kMaxK];
    float ts[kMaxK];
    route_select(a, sc, ids, ts);
    return finish_route(a, ids, ts);
}

// Routing of 4 tokens per wave, one per 16-lane row: lane p of a row holds
// the token's scores p, p + 16, ... (experts past n_experts are never
// selected). k rounds of a row-wide max pick the selected experts as
// top_k_distinct64 does, all rows at once; a row whose k largest scores are
// not distinct and strictly above the rest, or that holds a NaN, is routed
// by math.topK's heap over the token's scores in memory instead (exact
// insertion order), by the row's first lane. t is the row's token; rows with
// t >= n_tokens do nothing useful.
__device__ __forceinline__ uint32_t row_max16u(uint32_t v) {
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xF, 0xF, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xF, 0xF, false));
    return max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xF, 0xF, false));
}

__device__ __forceinline__ int row_max16i(int v) {
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false));
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false));
    v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false));
    return max(v, __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false));
}

// NC score slots per lane: lane p of a row holds experts p + 16 c, c < NC
// (NC = 4 covers 64 experts, 16 covers 256). Each of the k rounds takes the
// row's largest remaining key (order_key) and is clean when exactly one live
// score of the row equals it as a float; the k picks of clean rounds are
// distinct and above every other score, which is math.topK's result.
template <int NC>
__device__ inline TokenRoute route_row16(const RouteArgs& a, uint32_t t) {
    const uint32_t lane = threadIdx.x & 63, p = lane & 15, row = lane >> 4;
    const uint32_t E = a.n_experts, k = a.k;
    const bool live = t < a.n_tokens;
    const BufRsrc sr = make_rsrc(a.scores + (uint64_t)(live ? t : 0) * E, live ? E * 4 : 0);
    float sc[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) sc[c] = __uint_as_float(buf_load_b32(sr, (p + 16 * c) * 4, 0));
    int key[NC];
    bool bad = false;
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const bool v = p + 16 * c < E;
        bad |= v && sc[c] != sc[c];
        key[c] = v ? order_key(sc[c]) : kKeyNone;
    }
    uint32_t ids[kMaxK] = {0, 0, 0, 0};
    float ts[kMaxK] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (uint32_t r = 0; r < kMaxK; ++r) {  // constant r: ids / ts stay in registers
        if (r >= k) break;
        int lk = key[0];
#pragma unroll
        for (int c = 1; c < NC; ++c) lk = max(lk, key[c]);
        const float m = key_float(row_max16i(lk));
        uint32_t hits = 0, hc = 0;
#pragma unroll
        for (int c = 0; c < NC; ++c)
            if (key[c] != kKeyNone && sc[c] == m) {
                ++hits;
                hc = c;
            }
        const unsigned long long who = __ballot(hits != 0);
        const uint32_t in_row = (uint32_t)(who >> (16 * row)) & 0xFFFFu;
        if (__builtin_popcount(in_row) != 1 || hits > 1) bad = true;
        ids[r] = row_max16u(hits ? p + 16 * hc + 1 : 0u) - 1u;
        ts[r] = m;
#pragma unroll
        for (int c = 0; c < NC; ++c)
            if (hits && hc == (uint32_t)c) key[c] = kKeyNone;
    }
    // A row is bad when any of its lanes saw a clash.
    const unsigned long long bad_rows = __ballot(bad);
    if ((bad_rows >> (16 * row)) & 0xFFFFu) {
        // Exact heap over the token's scores, by the row's first lane.
        if (p == 0 && live) {
            const float* srow = a.scores + (uint64_t)t * E;
            top_k_heap([&](uint32_t j) { return srow[j]; }, E, k, ids, ts);
        }
        // Row-uniform again: lane 16 row holds the result.
#pragma unroll
        for (int i = 0; i < kMaxK; ++i) {
            ids[i] = (uint32_t)__shfl((int)ids[i], (int)(16 * row), 64);
            ts[i] = __shfl(ts[i], (int)(16 * row), 64);
        }
    }
    return finish_route(a, ids, ts);
}

__device__ inline TokenRoute route_token(const RouteArgs& a, uint32_t t) {
    float sc[4];
    load_scores(a, t, sc);
    return route_scores(a, sc);
}

// The routing outputs of a decode call (the single-token branch of the
// routing kernel): route ids / weights, statistics, slots in route order,
// the shared slot, and the down problem list. One thread.
__device__ inline void decode_route_outputs(const RouteArgs& a, const TokenRoute& tr) {
    const uint32_t E = a.n_experts, k = a.k;
#pragma unroll
    for (uint32_t i = 0; i < kMaxK; ++i) {
        if (a.route_ids) a.route_ids[i] = i < k ? tr.ids[i] : 0xFFFFFFFFu;
        if (a.route_w) a.route_w[i] = i < k ? tr.w[i] : 0.0f;
        a.assign_w[i] = ((tr.act >> i) & 1u) ? tr.w[i] : 0.0f;
        a.assign_slot[i] = -1;
    }
#pragma unroll
    for (uint32_t i = 0; i < kMaxK; ++i)
        if (i < k) atomicAdd(a.counts + tr.ids[i], 1ull);  // stats.record
    a.deferred[0] = tr.deferred;
    a.shared_slot[0] = a.shared ? 4 : -1;
    a.slot_tok[4] = 0;
    uint32_t s = 0;
#pragma unroll
    for (uint32_t i = 0; i < kMaxK; ++i) {
        if (i >= k || !((tr.act >> i) & 1u)) continue;
        a.assign_slot[i] = (int32_t)s;
        a.slot_tok[s] = 0;
        a.gemv_gu[2 * s] = make_uint4(tr.ids[i], 0, 2 * s, 0);
        a.gemv_gu[2 * s + 1] = make_uint4(E + tr.ids[i], 0, 2 * s + 1, 0);
        a.gemv_dn[s] = make_uint4(tr.ids[i], s, s, 0);
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

}  // namespace mmhip
