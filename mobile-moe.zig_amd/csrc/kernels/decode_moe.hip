// One-launch decode MoE layer for IQ2_XXS experts on gfx950: moeFFN for one
// token (inference.zig:886-1010) with the router matVecMul (math.zig:79-99,
// called at inference.zig:903), Scheduler.route (scheduler.zig:169-262),
// expertFFN (inference.zig:1152-1188) over the routed experts and the merged
// shared expert, and the weighted combine, in a single launch of one
// 1024-thread workgroup per CU.
//
// At one token the layer is a chain of short dependent steps (router scores ->
// routing -> gate/up -> down -> sum), each moving a few MB: as separate
// launches every step pays a launch ramp, a first-load latency and a drain.
// Here the steps hand over inside the launch:
//
//   1. E workgroups (the first ones without a shared-expert job) compute one
//      router row each in math.matVecMul's summation order (as
//      gemv_strict_kernel does) and publish the score.
//      Meanwhile every workgroup loads the IQ2_XXS tables and quantises the
//      hidden vector into LDS, and the shared expert's gate/up jobs (which do
//      not depend on the routing) are computed.
//   2. Each workgroup waits for all E scores and routes the token itself
//      (identical routing everywhere; workgroup 0 also writes the routing
//      outputs). It then issues its routed gate/up job's weight loads and,
//      right behind them, its down tile's weight loads for every problem, so
//      the down projection's memory latency overlaps the gate/up work.
//   3. A job is 32 rows of one problem's gate and up matrices: it forms
//      h = silu(gate) * up for one 32-element block of the down input,
//      quantises it to the down GEMV's digit planes and publishes them.
//   4. Down workgroup t waits for every job, copies every problem's h planes
//      into LDS, multiplies its prefetched row tile t of every problem's down
//      matrix, and sums the tile's rows over the problems in route order
//      (shared last, deferral bias after), as the separate down and combine
//      launches do.
//
// Every product, row sum, activation and combine uses the same arithmetic in
// the same order as the three-launch path (gemv_strict_kernel, the routing
// gate/up GEMV and down_combine_iq2_kernel), so the output is bit-identical
// to it.
//
// Hand-over between workgroups (each XCD has its own L2) without atomics or
// cache-wide fences. The host numbers the layer's calls (epoch, never 0):
//   - a score is published as one 64-bit device-scope (sc1) store of
//     (epoch << 32 | score bits), so one device-scope load returns both the
//     value and whether it belongs to this call;
//   - an h block is written with device-scope stores; once they are performed
//     (s_waitcnt vmcnt(0)), its flag word is set to the epoch. Consumers poll
//     the flags with device-scope loads and then read the blocks' digit
//     planes and scales with device-scope loads too, so no line another
//     XCD wrote is served stale from this XCD's L2.
// The memory model's agent-scope release/acquire fences write back and
// invalidate the whole L2 per use, and a single shared counter serialises
// hundreds of atomics; both cost several microseconds per hand-over here.
// A plain launch needs every workgroup resident at once (one per CU), which
// holds on a device no other kernel occupies; a launch that cannot become
// resident fails instead of hanging: a wait gives up after a bounded time
// and records the failure in a host-visible status word, so a launch
// always ends.
#include "iq2_ops.hpp"
#include "kernels.hpp"
#include "route_ops.hpp"

namespace mmhip {

namespace {

constexpr int kDmWg = 1024;
constexpr uint32_t kDmWaves = kDmWg / 64;
constexpr uint32_t kDmMaxProbs = kMaxK + 1;    // routed + shared
constexpr uint32_t kDmMaxUnits = 8;            // hidden, inter <= 2048
constexpr uint32_t kDmJobItems = 2 * 2 * kDmMaxUnits;  // gate and up, two row tiles, every unit
constexpr uint32_t kDmJobPerWave = kDmJobItems / kDmWaves;
constexpr uint32_t kDmDownItems = kDmMaxProbs * kDmMaxUnits;
// Down items run on waves 1..15: wave 0 publishes the h blocks, and its
// s_waitcnt for those stores would also wait for any weight loads it had
// issued before them.
constexpr uint32_t kDmDownWaves = kDmWaves - 1;
constexpr uint32_t kDmDownPerWave = (kDmDownItems + kDmDownWaves - 1) / kDmDownWaves;
constexpr uint32_t kDmMaxHBlocks = kDmMaxProbs * kDmMaxUnits * 8;  // 32-element blocks of every problem's h
constexpr uint32_t kDmRouterRow = kDmMaxUnits * 256 / 4 + 4;        // one chain's terms, padded (banks)

static_assert(kDmJobItems % kDmWaves == 0, "job items split evenly over the waves");

struct DmLds {
    uint32_t tab[kIq2TableWords];
    uint32_t mtab[8];
    uint8_t xq[kDmMaxUnits * 8 * 64];  // hidden vector digit planes
    float xs[kDmMaxUnits * 8];
    float prod[4][kDmRouterRow];       // router products, one row per chain
    float rows_gu[kDmJobItems * 16];   // each job item's 16 row values
    float hrow[64];                    // gate rows 0..31, up rows 0..31 of a job
    uint8_t hq[kDmMaxHBlocks * 64];    // every problem's h planes (down input)
    float hs[kDmMaxHBlocks];
    float rows_dn[kDmDownItems * 16];
    float ysum[kDmMaxProbs * 16];
    uint32_t route[2 + 2 * kMaxK];     // act, deferred, ids, weight bits
    uint32_t route_e[kMaxK];           // computed routed experts in route order
    uint32_t route_n;                  // their count
};

// Device-scope store of one published word.
__device__ __forceinline__ void publish_u32(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Bounded wait (one wave): load(v) issues one round of device-scope loads
// into v, done(v) tells whether everything it read is published. One round
// is in flight at a time: a second one issued ahead would still be in
// flight on return, and the next use of its registers would wait for it.
// The wait is bounded by time, read from the constant 100 MHz real-time
// counter (s_memrealtime, 10 ns per tick): once `ticks` have passed since
// the first poll (0: after the first poll), it gives up and records `code`.
template <typename V, typename Load, typename Done>
__device__ __forceinline__ void grid_wait(V& v, Load load, Done done, uint32_t ticks, uint32_t* status,
                                          uint32_t code) {
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    for (;;) {
        load(v);
        if (done(v)) return;
        if (__builtin_amdgcn_s_memrealtime() - t0 >= ticks) {
            if (status) __hip_atomic_store(status, code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            return;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// Router row in math.matVecMul's order (the arithmetic of
// gemv_strict_kernel<WT, 1>, columns a multiple of 16): thread i < cols / 4
// holds column quad i of the row (w4, or h4 for f16 weights) and of the
// hidden vector (x4). Products are de-interleaved into prod[l][i] =
// w[4 i + l] * x[4 i + l], four chains l sum their terms in column order and
// the score is ((a0 + a1) + a2) + a3. Every thread takes part (LDS barriers
// inside); thread 0 returns the score.
__device__ float router_row(bool f16, const uint4& w4, const uint2& h4, const uint4& x4, uint32_t cols,
                            float (*prod)[kDmRouterRow]) {
#pragma clang fp contract(off)
    const uint32_t tid = threadIdx.x;
    if (tid < cols / 4) {
        float wv[4];
        if (f16) {
            wv[0] = f16_bits_to_f32(h4.x & 0xFFFFu);
            wv[1] = f16_bits_to_f32(h4.x >> 16);
            wv[2] = f16_bits_to_f32(h4.y & 0xFFFFu);
            wv[3] = f16_bits_to_f32(h4.y >> 16);
        } else {
            wv[0] = __uint_as_float(w4.x);
            wv[1] = __uint_as_float(w4.y);
            wv[2] = __uint_as_float(w4.z);
            wv[3] = __uint_as_float(w4.w);
        }
        prod[0][tid] = wv[0] * __uint_as_float(x4.x);
        prod[1][tid] = wv[1] * __uint_as_float(x4.y);
        prod[2][tid] = wv[2] * __uint_as_float(x4.z);
        prod[3][tid] = wv[3] * __uint_as_float(x4.w);
    }
    lds_barrier();
    float acc = 0.0f;
    if (tid < 4) {
        // Batches of 32 terms read into two register sets in turn, so the
        // next batch's LDS reads are in flight while the current one is added.
        const float4* pp = reinterpret_cast<const float4*>(&prod[tid][0]);
        const uint32_t n16 = cols / 16, nb = n16 / 8;
        float4 ra[8], rb[8];
        auto read = [&](float4 (&r)[8], uint32_t b) {
#pragma unroll
            for (int k = 0; k < 8; ++k) r[k] = pp[b * 8 + k];
            __builtin_amdgcn_sched_barrier(0);
        };
        auto add = [&](const float4 (&r)[8]) {
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                acc = acc + r[k].x;
                acc = acc + r[k].y;
                acc = acc + r[k].z;
                acc = acc + r[k].w;
            }
        };
        uint32_t b = 0;
        if (nb > 0) read(ra, 0);
        for (; b + 2 <= nb; b += 2) {
            read(rb, b + 1);
            add(ra);
            read(ra, min(b + 2, nb - 1));
            add(rb);
        }
        if (b < nb) add(ra);
        for (uint32_t i = nb * 8; i < n16; ++i) {
            const float4 t = pp[i];
            acc = acc + t.x;
            acc = acc + t.y;
            acc = acc + t.z;
            acc = acc + t.w;
        }
    }
    const float a1 = __shfl_down(acc, 1, kWave), a2 = __shfl_down(acc, 2, kWave), a3 = __shfl_down(acc, 3, kWave);
    return ((acc + a1) + a2) + a3;
}

__global__ __launch_bounds__(kDmWg, 1) void decode_moe_iq2_kernel(DecodeMoeArgs a) {
    __shared__ __align__(16) DmLds lds;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t n = lane & 15, g = lane >> 4;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t w = blockIdx.x, G = gridDim.x;
    const uint32_t E = a.route.n_experts;
    const uint32_t epoch = a.epoch;
    const uint32_t hu = a.hidden / 256;   // gate/up record units per row tile
    const uint32_t du = a.inter / 256;    // down record units per row tile
    const uint32_t nbh = a.inter / 32;    // h blocks (jobs) per problem
    const uint32_t dn_tiles = a.hidden / 16;
    const uint32_t sh = a.route.shared ? 1u : 0u;  // problem 0 is the shared expert when present

    // ---- Router row loads first (the routing waits on them): row r on
    // workgroup r0 + r, the first workgroups without a shared-expert job
    // (vector loads return in issue order, so a job's weight loads would
    // hold the row's loads back). Workgroups are dispatched in id order, so
    // low ids start earliest: 0.3 us per token sooner than on the last E.
    // Other workgroups' resources are empty (the loads read zeros without a
    // memory access), so every load is issued unconditionally and the
    // compiler's load counters stay exact.
    const uint32_t r0 = G >= sh * nbh + E ? sh * nbh : G - E;
    const bool router_wg = w >= r0 && w < r0 + E;
    const uint32_t r_row = router_wg ? w - r0 : 0;
    const bool f16_router = a.router_type != 0;
    const uint32_t rbytes = router_wg ? a.hidden * (f16_router ? 2u : 4u) : 0u;
    const char* rrow = static_cast<const char*>(a.router_w) + (uint64_t)r_row * a.hidden * (f16_router ? 2u : 4u);
    const uint4 rw4 = buf_load_b128(make_rsrc(rrow, f16_router ? 0u : rbytes), threadIdx.x * 16, 0);
    const uint2 rh4 = buf_load_b64(make_rsrc(rrow, f16_router ? rbytes : 0u), threadIdx.x * 8, 0);
    const uint4 rx4 = buf_load_b128(make_rsrc(a.x, router_wg ? a.hidden * 4 : 0u), threadIdx.x * 16, 0);

    // ---- Small loads: tables and the hidden vector.
    const BufRsrc t_r = make_rsrc(&c_iq2_tables, sizeof(Iq2Tables));
    uint4 tv[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) tv[i] = buf_load_b128(t_r, (threadIdx.x + kDmWg * i) * 16, 0);
    float xv[4];
    x_pass_load(make_rsrc(a.x, a.hidden * 4), 0, xv);  // 128 blocks per pass >= hidden / 32

    // Whole-stack resources: matrix mat of a stack starts mat * (matrix
    // bytes) in (the stacks are below 2 GiB, checked at launch), so once the
    // routing names a matrix a load needs one scalar multiply-add.
    const uint32_t gu_mb = (uint32_t)(a.gu_rec_stride * 16), gu_db = (uint32_t)(a.gu_d_stride * 2);
    const uint32_t dn_mb = (uint32_t)(a.dn_rec_stride * 16), dn_db = (uint32_t)(a.dn_d_stride * 2);
    const uint32_t n_gu_mats = 2 * E + 2 * sh, n_dn_mats = E + sh;
    const BufRsrc gu_r = make_rsrc(a.gu_recs, n_gu_mats * gu_mb);
    const BufRsrc gud_r = make_rsrc(a.gu_dvals, n_gu_mats * gu_db);
    const BufRsrc dn_r = make_rsrc(a.dn_recs, n_dn_mats * dn_mb);
    const BufRsrc dnd_r = make_rsrc(a.dn_dvals, n_dn_mats * dn_db);

    // Gate/up job j: problem p = j / nbh, h block b = j % nbh (rows 32 b ..
    // 32 b + 31 of the gate and up matrices). Item i = (m * 2 + tt) * hu + u
    // (m: gate 0 / up 1, tt: row tile 2 b + tt, u: unit) runs on wave
    // i % 16, register slot i / 16; its offsets within its matrix depend on
    // b only. Loads are issued unconditionally (slots past the job read
    // zeros without a memory access), so the compiler's load counters stay
    // exact.
    const uint32_t n_job_items = 4 * hu;
    struct JobSlots {
        uint32_t rec[kDmJobPerWave], d[kDmJobPerWave];
        bool up[kDmJobPerWave], ok[kDmJobPerWave];
    };
    auto job_slots = [&](uint32_t b) {
        JobSlots js;
#pragma unroll
        for (uint32_t s = 0; s < kDmJobPerWave; ++s) {
            const uint32_t i = wave + kDmWaves * s;
            const uint32_t m = i / (2 * hu), rest = i - m * 2 * hu, tt = rest / hu, u = rest - tt * hu;
            const uint32_t tile = 2 * b + tt;
            js.rec[s] = (tile * hu + u) * 1024;
            js.d[s] = (tile * 16 * a.gu_d_row + u) * 2;
            js.up[s] = m != 0;
            js.ok[s] = i < n_job_items;
        }
        return js;
    };
    auto job_issue = [&](bool run, uint32_t gate_mat, uint32_t up_mat, const JobSlots& js,
                         uint4 (&rb)[kDmJobPerWave], uint16_t (&db)[kDmJobPerWave]) {
#pragma unroll
        for (uint32_t s = 0; s < kDmJobPerWave; ++s) {
            const uint32_t mat = js.up[s] ? up_mat : gate_mat;
            const bool ok = run && js.ok[s];
            rb[s] = buf_load_b128<kCacheStream>(gu_r, lane * 16, ok ? mat * gu_mb + js.rec[s] : kBufOob);
            db[s] = buf_load_b16(gud_r, n * a.gu_d_row * 2, ok ? mat * gu_db + js.d[s] : kBufOob);
        }
    };
    // Items of a job (every wave): each item's 16 row values, lane groups
    // summed in order in registers.
    auto job_items = [&](const uint4 (&rb)[kDmJobPerWave], const uint16_t (&db)[kDmJobPerWave]) {
#pragma unroll
        for (uint32_t s = 0; s < kDmJobPerWave; ++s) {
            const uint32_t i = wave + kDmWaves * s;
            if (i < n_job_items) {
                const uint32_t u = i % hu;
                const float v =
                    item_rows(iq2_item(rb[s], db[s], lds.xq + u * 8 * 64, lds.xs + u * 8, lds.tab, lds.mtab, n, g));
                if (lane < 16) lds.rows_gu[i * 16 + lane] = v;
            }
        }
        lds_barrier();
    };
    // Row sums of the job (units in order, as the decode GEMV sums a row),
    // h = silu(gate) * up, quantised as the down GEMV quantises its input,
    // published for every down workgroup. Wave 0 only.
    auto job_publish = [&](uint32_t p, uint32_t b) {
        // Lane l < 32: gate row l of the block; lane 32 + l: up row l.
        const uint32_t m = lane >> 5, r = lane & 31, tt = r >> 4, rr = r & 15;
        float sum = 0.0f;
        for (uint32_t u = 0; u < hu; ++u) sum += lds.rows_gu[((m * 2 + tt) * hu + u) * 16 + rr];
        lds.hrow[lane] = 0.0f + sum;
        // Lane jq < 8 takes rows 4 jq .. 4 jq + 3 (every lane joins the
        // block maxima; lanes >= 8 quantise a copy and store nothing). The
        // wave's own LDS writes above are visible to its reads in order.
        const uint32_t jq = lane & 7;
        const float4 gr = *reinterpret_cast<const float4*>(lds.hrow + 4 * jq);
        const float4 ur = *reinterpret_cast<const float4*>(lds.hrow + 32 + 4 * jq);
        float v[4] = {silu_fast(gr.x) * ur.x, silu_fast(gr.y) * ur.y, silu_fast(gr.z) * ur.z, silu_fast(gr.w) * ur.w};
        uint32_t h4, l4;
        const float scale = quantize_quad(v, h4, l4);
        const uint32_t blk = p * nbh + b;
        if (lane < 8) {
            publish_u32(reinterpret_cast<uint32_t*>(a.hq + (uint64_t)blk * 64 + 4 * jq), h4);
            publish_u32(reinterpret_cast<uint32_t*>(a.hq + (uint64_t)blk * 64 + 32 + 4 * jq), l4);
            if (lane == 0) publish_u32(reinterpret_cast<uint32_t*>(a.hs + blk), __float_as_uint(scale));
        }
        // The flag once the block's stores are performed (stores count in
        // vmcnt on gfx950).
        __builtin_amdgcn_s_waitcnt(0x0F70);
        if (lane == 0) publish_u32(a.h_flags + blk, epoch);
    };

    // ---- The shared expert's first job needs no routing: its loads go out
    // now, behind every wave's small loads.
    uint4 rb_gu[kDmJobPerWave];
    uint16_t db_gu[kDmJobPerWave];
    const bool shared_job = sh && w < nbh;
    __builtin_amdgcn_s_barrier();
    job_issue(shared_job, 2 * E, 2 * E + 1, job_slots(w), rb_gu, db_gu);
    if (router_wg) {
        const float score = router_row(f16_router, rw4, rh4, rx4, a.hidden, lds.prod);
        if (threadIdx.x == 0)
            __hip_atomic_store(a.score_tags + r_row, ((uint64_t)epoch << 32) | __float_as_uint(score),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) reinterpret_cast<uint4*>(lds.tab)[threadIdx.x + kDmWg * i] = tv[i];
    if (threadIdx.x < 8) lds.mtab[threadIdx.x] = iq2_hi3_mask(threadIdx.x);
    x_store_planes(xv, hu * 8, 0, lds.xq, lds.xs);
    lds_barrier();  // tables and hidden planes visible
    if (shared_job) {
        job_items(rb_gu, db_gu);
        if (wave == 0) job_publish(0, w);
    }

    // What the routed loads need apart from the routing, worked out while
    // the router rows are computed: this workgroup's routed job (j_r, its
    // problem p_r and block b_r) and down tile slots. Down item
    // i = p * du + u runs on wave 1 + i % 15, slot i / 15.
    const uint32_t j_r = w + (shared_job ? G : 0);
    const uint32_t p_r = j_r / nbh, b_r = j_r - p_r * nbh;
    const JobSlots js_r = job_slots(b_r);
    const uint32_t dt = w;  // down row tile (dn_tiles <= grid)
    uint32_t dn_rec[kDmDownPerWave], dn_d[kDmDownPerWave], dn_p[kDmDownPerWave];
#pragma unroll
    for (uint32_t s = 0; s < kDmDownPerWave; ++s) {
        const uint32_t i = (wave - 1) + kDmDownWaves * s;
        const bool ok = wave > 0 && dt < dn_tiles && i < kDmMaxProbs * du;
        const uint32_t p = ok ? i / du : kDmMaxProbs, u = ok ? i - p * du : 0;
        dn_p[s] = p;
        dn_rec[s] = (dt * du + u) * 1024;
        dn_d[s] = (dt * 16 * a.dn_d_row + u) * 2;
    }

    // ---- Routing, by wave 0 of every workgroup: scores e = lane + 64 q
    // (experts past E read as published zeros and are never selected). The
    // selected ids and which of them are computed go to every wave at once;
    // the route weights (softmax over the selected logits), needed only by
    // the combine, follow while the weight loads are in flight.
    uint32_t r_ids[kMaxK];
    float r_ts[kMaxK];
    if (wave == 0) {
        struct Tags {
            uint64_t v[4];
        } ta;
        const uint64_t none = (uint64_t)epoch << 32;
        grid_wait(
            ta,
            [&](Tags& t) {
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const uint32_t e = lane + 64 * q;
                    t.v[q] = e < E ? __hip_atomic_load(a.score_tags + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                   : none;
                }
            },
            [&](const Tags& t) {
                bool ok = true;
#pragma unroll
                for (int q = 0; q < 4; ++q) ok = ok && (uint32_t)(t.v[q] >> 32) == epoch;
                return __all(ok) != 0;
            },
            a.wait_ticks, a.status, 1u);
        float sc[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) sc[q] = __uint_as_float((uint32_t)ta.v[q]);
        route_select(a.route, sc, r_ids, r_ts);
        uint32_t act, deferred;
        route_active(a.route, act, deferred);
        if (lane == 0) {
            uint32_t na = 0;
#pragma unroll
            for (uint32_t i = 0; i < kMaxK; ++i) {
                lds.route[2 + i] = r_ids[i];
                if (i < a.route.k && ((act >> i) & 1u)) lds.route_e[na++] = r_ids[i];
            }
            lds.route[0] = act;
            lds.route[1] = deferred;
            lds.route_n = na;
        }
    }
    lds_barrier();
    const uint32_t k = a.route.k;
    const uint32_t act = lds.route[0], deferred = lds.route[1];
    // Problems: the shared expert (p = 0, when present), then the computed
    // routed experts in route order (route_e).
    const uint32_t P = sh + lds.route_n, n_jobs = P * nbh;

    // ---- Routed gate/up job loads, then this workgroup's down tile loads.
    {
        const bool run = j_r < n_jobs;
        const uint32_t e = lds.route_e[run ? p_r - sh : 0];
        job_issue(run, e, E + e, js_r, rb_gu, db_gu);
    }
    if (wave == 0) {
        // The route weights (read by the combine, after later barriers) and,
        // by workgroup 0, the routing outputs.
        const TokenRoute tr = finish_route(a.route, r_ids, r_ts);
        if (w == 0 && lane == 0) decode_route_outputs(a.route, tr);
        if (lane == 0) {
#pragma unroll
            for (uint32_t i = 0; i < kMaxK; ++i) lds.route[2 + kMaxK + i] = __float_as_uint(tr.w[i]);
        }
    }
    // The job's items, then wave 0 publishes h, then waves 1..15 issue the
    // down tile's loads (needed only after the next hand-over). A CU takes
    // vector memory instructions in issue order, so down loads issued
    // earlier would hold back the job's data and wave 0's h stores; and
    // wave 0 issues none, so its wait for its h stores waits for nothing
    // else.
    const bool run_r = j_r < n_jobs;
    if (run_r) job_items(rb_gu, db_gu);
    if (wave == 0 && run_r) job_publish(p_r, b_r);
    __builtin_amdgcn_s_barrier();
    uint4 rb_dn[kDmDownPerWave];
    uint16_t db_dn[kDmDownPerWave];
    const uint32_t n_dn_items = P * du;
    if (wave != 0) {
#pragma unroll
        for (uint32_t s = 0; s < kDmDownPerWave; ++s) {
            const uint32_t p = dn_p[s];
            const bool ok = p < P;
            const uint32_t mat = ok ? ((sh && p == 0) ? E : lds.route_e[p - sh]) : 0;
            rb_dn[s] = buf_load_b128<kCacheStream>(dn_r, lane * 16, ok ? mat * dn_mb + dn_rec[s] : kBufOob);
            db_dn[s] = buf_load_b16(dnd_r, n * a.dn_d_row * 2, ok ? mat * dn_db + dn_d[s] : kBufOob);
        }
    }
    // Further jobs (more jobs than workgroups) load after the first.
    for (uint32_t j = j_r + G; j < n_jobs; j += G) {
        const uint32_t p = j / nbh, b = j - p * nbh;
        const uint32_t e = lds.route_e[p - sh];
        lds_barrier();  // rows_gu free
        job_issue(true, e, E + e, job_slots(b), rb_gu, db_gu);
        job_items(rb_gu, db_gu);
        if (wave == 0) job_publish(p, b);
    }

    // ---- Down projection and combine of row tile dt.
    if (dt < dn_tiles) {
        auto stage = [&](uint32_t j0, uint32_t j1) {
            // Jobs [j0, j1) (whole problems): wait for their flags (wave 0),
            // copy their h planes and scales into LDS, then the down items of
            // their problems. Planes and scales are read with device-scope
            // loads, which miss in this XCD's L2 for lines another XCD
            // wrote: the flag loads above are relaxed, so nothing else
            // orders a plain load after the writer's stores, and a line
            // cached before them (a scale line holds several problems'
            // scales) would be stale.
            if (wave == 0) {
                constexpr int kQ = (kDmMaxHBlocks + 63) / 64;  // flags per lane, at most
                struct Flags {
                    uint32_t v[kQ];
                } fa;
                grid_wait(
                    fa,
                    [&](Flags& f) {
#pragma unroll
                        for (int q = 0; q < kQ; ++q) {
                            const uint32_t jj = j0 + lane + 64 * q;
                            f.v[q] = jj < j1 ? __hip_atomic_load(a.h_flags + jj, __ATOMIC_RELAXED,
                                                                 __HIP_MEMORY_SCOPE_AGENT)
                                             : epoch;
                        }
                    },
                    [&](const Flags& f) {
                        bool ok = true;
#pragma unroll
                        for (int q = 0; q < kQ; ++q) ok = ok && f.v[q] == epoch;
                        return __all(ok) != 0;
                    },
                    a.wait_ticks, a.status, 2u);
            }
            lds_barrier();
            const BufRsrc qr = make_rsrc(a.hq + (uint64_t)j0 * 64, (j1 - j0) * 64);
            for (uint32_t o = threadIdx.x * 16; o < (j1 - j0) * 64; o += kDmWg * 16)
                *reinterpret_cast<uint4*>(lds.hq + j0 * 64 + o) = buf_load_b128<kCacheDevice>(qr, o, 0);
            const BufRsrc sr = make_rsrc(a.hs + j0, (j1 - j0) * 4);
            if (threadIdx.x < j1 - j0)
                lds.hs[j0 + threadIdx.x] = __uint_as_float(buf_load_b32<kCacheDevice>(sr, threadIdx.x * 4, 0));
            lds_barrier();
            // Items i = p * du + u of these jobs' problems (j0, j1 are whole
            // problems: multiples of nbh = 8 du).
            const uint32_t i0 = j0 / 8, i1 = j1 / 8;
#pragma unroll
            for (uint32_t s = 0; s < kDmDownPerWave; ++s) {
                const uint32_t i = (wave - 1) + kDmDownWaves * s;
                if (wave > 0 && i >= i0 && i < i1) {
                    const float v = item_rows(
                        iq2_item(rb_dn[s], db_dn[s], lds.hq + i * 8 * 64, lds.hs + i * 8, lds.tab, lds.mtab, n, g));
                    if (lane < 16) lds.rows_dn[i * 16 + lane] = v;
                }
            }
        };
        stage(0, n_jobs);
        lds_barrier();
        if (threadIdx.x < 16 * P) {
            // Row r of problem p: the decode GEMV's row sum (units in order).
            const uint32_t p = threadIdx.x >> 4, r = threadIdx.x & 15;
            float sum = 0.0f;
            for (uint32_t u = 0; u < du; ++u) sum += lds.rows_dn[(p * du + u) * 16 + r];
            lds.ysum[p * 16 + r] = 0.0f + sum;
        }
        lds_barrier();
        const uint32_t row = dt * 16 + threadIdx.x;
        if (threadIdx.x < 16 && row < a.hidden) {
            // Computed assignments in route order, then the shared expert,
            // then the deferral bias (combine_kernel's order).
            float o = 0.0f;
            uint32_t q = sh;
#pragma unroll
            for (uint32_t i = 0; i < kMaxK; ++i) {
                if (i < k && ((act >> i) & 1u)) {
                    o = __fadd_rn(o, __fmul_rn(__uint_as_float(lds.route[2 + kMaxK + i]), lds.ysum[q * 16 + threadIdx.x]));
                    ++q;
                }
            }
            if (sh) o = __fadd_rn(o, lds.ysum[threadIdx.x]);
            if (a.bias && deferred) o = __fadd_rn(o, a.bias[row]);
            a.out[row] = o;
        }
    }
}

}  // namespace

bool decode_moe_iq2_fits(uint32_t hidden, uint32_t inter, uint32_t n_experts, int num_cu) {
    const uint32_t G = (uint32_t)(num_cu > 0 ? num_cu : 0);
    if (hidden % 256 || inter % 256 || hidden < 256 || inter < 256 || hidden / 256 > kDmMaxUnits ||
        inter / 256 > kDmMaxUnits || n_experts < 1 || n_experts > 256 || n_experts > G || hidden / 16 > G ||
        inter / 32 > G)
        return false;
    // Whole stacks addressed through one buffer resource each, with 32-bit
    // offsets below kBufOob: (2E + 2) gate/up and (E + 1) down matrices.
    const uint64_t mat_bytes = (uint64_t)(hidden / 256) * (inter / 16) * 1024;  // both shapes
    return (uint64_t)(2 * n_experts + 2) * mat_bytes < kBufOob;
}

hipError_t launch_decode_moe_iq2(const DecodeMoeArgs& a, int num_cu, hipStream_t s) {
    const uint32_t E = a.route.n_experts, sh = a.route.shared ? 1u : 0u;
    if (!decode_moe_iq2_fits(a.hidden, a.inter, E, num_cu) || a.route.n_tokens != 1 ||
        (2 * E + 2 * sh) * a.gu_rec_stride * 16 >= kBufOob || (E + sh) * a.dn_rec_stride * 16 >= kBufOob ||
        (2 * E + 2 * sh) * a.gu_d_stride * 2 >= kBufOob || (E + sh) * a.dn_d_stride * 2 >= kBufOob ||
        a.route.k < 1 || a.route.k > kMaxK || (a.route.shared && !a.route.shared_merged) || a.epoch == 0)
        return hipErrorInvalidValue;
    DecodeMoeArgs args = a;
    void* kargs[] = {&args};
    static const bool coop = [] {
        const char* e = getenv("MMHIP_DECODE_COOP");
        return e && e[0] == '1';
    }();
    if (coop)
        return hipLaunchCooperativeKernel(reinterpret_cast<const void*>(&decode_moe_iq2_kernel),
                                          dim3((uint32_t)num_cu), dim3(kDmWg), kargs, 0, s);
    return hipLaunchKernel(reinterpret_cast<const void*>(&decode_moe_iq2_kernel), dim3((uint32_t)num_cu), dim3(kDmWg),
                           kargs, 0, s);
}

}  // namespace mmhip
