// Decode GEMV on gfx950.
//
// Q8_0 weights: a workgroup (one per CU) owns one activation vector
// (problem) and a contiguous range of 16-row tiles. It quantises the vector
// into LDS (the A operand of every MFMA, so the separate quantisation launch
// disappears), and its waves then stream equal shares of the range's 1 KiB
// record units, one 128-bit load per lane, steps ahead of the compute. Every
// weight byte is read exactly once. IQ2_XXS weights have their own kernel
// (gemv_iq2.hip); launch_gemv_q forwards them there.
//
// f32 / f16 weights (the router, matVecMulUnified's f32 branch): one
// workgroup per output row, summing in the reference's order
// (gemv_strict_kernel).
#include "device_common.hpp"
#include "kernels.hpp"
#include "route_ops.hpp"
#include "tile_ops.hpp"

#include <cstdlib>

namespace mmhip {

namespace {

constexpr uint32_t kChunkBlocks = 256;  // 8192 columns of activation per LDS chunk (multiple of 8)
constexpr uint32_t kGemvMaxTiles = 64;  // tiles per workgroup (LDS row sums)

// Position of a decode step: tile t (within the workgroup's range) and step s
// within the tile's part of the current K-chunk.
struct StepPos {
    uint32_t t, s;
};

// UPS = record units per step (compile-time); a tile's units in a K-chunk are
// a whole number of steps. WG threads per workgroup.
//
// Work split: a workgroup owns one problem's tiles [t_begin, t_begin + n_tiles)
// and, per K-chunk, its n_tiles * S steps (S steps per tile) are split into
// kWaves contiguous, equal runs, one per wave: the wave of step j is the
// largest w with floor(w * L / kWaves) <= j (L = n_tiles * S). A wave's run
// covers whole tiles and at most two partial ones (its first and last).
// Whole tiles add their row sums straight into the workgroup's LDS sums;
// partial tiles leave theirs in the wave's edge slots (0: its first tile,
// 1: its last), and after the chunk a combine pass adds each split tile's
// pieces in wave order, so results do not depend on timing.
//
// Loads: every weight, scale and activation load goes through a buffer
// resource and is issued unconditionally (out-of-range offsets for steps past
// the wave's end), so each wait covers exactly the loads it needs. A CU
// returns loads in issue order across its waves, and a wave cannot issue
// while the CU's load queue is full: weights issued before another wave's
// prologue loads would delay that wave's prologue. So every wave issues its
// table and activation loads, a barrier orders the issue, and only then do
// the first weight steps go out; the waits for the prologue data leave them
// in flight while LDS is filled. The stream runs one step ahead (two register
// buffers): the CU's queue holds about one step per wave, and a deeper
// prefetch only blocks the issuing wave.
template <int UPS, int WG, int DEPTH, bool ROUTE, int NSEG, class A>
__device__ __forceinline__ void gemv_q_body(const A& a, const GemvArgs& lt) {
    constexpr int FMT = kFmtQ8;
    constexpr uint32_t kWaves = WG / 64;
    constexpr int kRing = DEPTH + 1;  // register buffers: the step computing + DEPTH in flight
    // Static LDS for the row sums; dynamic LDS for the activation chunk.
    __shared__ float row_sum[kGemvMaxTiles * 16];
    __shared__ float edge[2][kWaves * 16];
    extern __shared__ __align__(16) uint8_t smem[];
    // a: this workgroup's segment; its problem is grid row y.
    const uint32_t t_begin = blockIdx.x * a.tiles_per_wg;
    // The grid is sized for the widest and longest segment.
    if (t_begin >= a.tiles || blockIdx.y >= a.n_probs) return;  // whole workgroup
    constexpr uint32_t kBlkPerUnit = 2;
    const uint32_t nblk_all = a.units * kBlkPerUnit;
    const uint32_t chunk_blk = nblk_all < kChunkBlocks ? nblk_all : kChunkBlocks;
    int8_t* aq = reinterpret_cast<int8_t*>(smem);
    float* xs = reinterpret_cast<float*>(smem + ((chunk_blk + 7) / 8) * kAGroupBytes);

    const uint32_t lane = threadIdx.x & 63;
    const uint32_t n = lane & 15, g = lane >> 4;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t p = blockIdx.y;
    uint64_t mat = a.first_mat + p, x_row = p, y_row = p;
    if constexpr (ROUTE) {
        // Every wave routes the token (same result); the problem follows.
        const TokenRoute tr = route_token(a.route, 0);
        if (p == 0 && blockIdx.x == 0 && threadIdx.x == 0) decode_route_outputs(a.route, tr);
        const uint32_t E = a.route.n_experts;
        uint32_t n_act = 0, e_sel = 0;
#pragma unroll
        for (uint32_t i = 0; i < kMaxK; ++i)
            if (i < a.route.k && ((tr.act >> i) & 1u)) {
                if (n_act == p >> 1) e_sel = tr.ids[i];
                ++n_act;
            }
        x_row = 0;
        if (p < 2 * n_act) {
            mat = (p & 1u) ? E + e_sel : e_sel;
        } else if (a.route.shared && a.route.shared_merged && p < 2 * n_act + 2) {
            mat = 2 * E + (p - 2 * n_act);
            y_row = 8 + (p - 2 * n_act);
        } else {
            return;  // whole workgroup: no such problem this call
        }
    } else {
        if (!read_problem(a.probs, a.n_active, p, mat, x_row, y_row)) return;  // whole workgroup: not in this call
    }
    const float* x = a.x + x_row * a.x_stride;
    float* const y_base = lt.y + y_row * lt.y_stride;
    const bool silu_mul = a.silu_mul != 0;
    const uint32_t n_tiles = min(a.tiles - t_begin, a.tiles_per_wg);
    const bool has_a = n < 2;
    const int8_t* a_run = aq + (n & 1) * 4 * kARun + g * kARun;  // used by lanes n < 2 only
    const float* xs_g = xs + g;
    const BufRsrc rec_r = make_rsrc(a.recs + mat * a.rec_stride, (uint32_t)(a.rec_stride * 16));
    const BufRsrc d_r = make_rsrc(a.dvals + mat * a.d_stride, (uint32_t)(a.d_stride * 2));
    const uint32_t rec_voff = lane * 16;
    const uint32_t d_voff = n * a.d_row * 2;
    const uint32_t rec_tile = keep_sgpr(a.units * 1024u), d_tile = keep_sgpr(a.d_row * 32u);

    // Per-chunk split (set by start_chunk).
    uint32_t u_begin = 0, S = 1, L = 0, j0 = 0, j1 = 0, tf = 0;
    auto start_chunk = [&](uint32_t nb) {
        S = (nb / kBlkPerUnit) / UPS;
        L = n_tiles * S;
        j0 = wave * L / kWaves;
        j1 = (wave + 1) * L / kWaves;
        tf = j0 / S;
    };
    auto advance = [&](StepPos q) { return (q.s + 1 == S) ? StepPos{q.t + 1, 0} : StepPos{q.t, q.s + 1}; };
    uint4 rb[kRing][kMaxUnitsPerStep];
    uint32_t db[kRing][kMaxUnitsPerStep];
    auto load = [&](bool valid, StepPos q, uint4 (&r)[kMaxUnitsPerStep], uint32_t (&dw)[kMaxUnitsPerStep]) {
        uint32_t rs = kBufOob, ds = kBufOob;
        if (valid) {
            const uint32_t t = t_begin + q.t, u = u_begin + q.s * UPS;
            rs = t * rec_tile + u * 1024;
            ds = t * d_tile + u * 4;
        }
        load_step<FMT, UPS>(rec_r, rec_voff, rs, d_r, d_voff, ds, r, dw);
    };
    float acc = 0.0f;
    bool seg_whole = true;  // the current tile segment started at the tile's first step
    StepPos cur{0, 0}, nxt{0, 0};  // the step to compute, the next to load
    // Issues the first DEPTH steps of the current chunk.
    auto issue_first = [&]() {
        cur = StepPos{tf, j0 - tf * S};
        nxt = cur;
        seg_whole = cur.s == 0;
#pragma unroll
        for (int q = 0; q < DEPTH; ++q) {
            load(j0 + q < j1, nxt, rb[q], db[q]);
            nxt = advance(nxt);
        }
    };
    // Computes step j (position q) from (r, dw); at the end of a tile segment
    // leaves the segment's row sums in LDS.
    auto compute = [&](uint32_t j, StepPos q, const uint4 (&r)[kMaxUnitsPerStep],
                       const uint32_t (&dw)[kMaxUnitsPerStep]) {
        const uint32_t ub = q.s * UPS;  // unit index within the LDS chunk
        step_dot_q8<UPS>(r, dw, ub, a_run, has_a, xs_g, g, acc);
        const bool tile_end = q.s + 1 == S;
        if (tile_end || j + 1 == j1) {
            const float tot = reduce_groups(acc);
            acc = 0.0f;
            if (lane < 16) {
                if (seg_whole && tile_end)
                    row_sum[q.t * 16 + n] += tot;
                else
                    edge[q.t == tf ? 0 : 1][wave * 16 + n] = tot;
            }
            seg_whole = true;
        }
    };

    {
        // Prologue: first activation chunk, zeroed row sums.
        const uint32_t nb = chunk_blk;
        const uint32_t xb = min(a.cols, chunk_blk * 32) * 4;
        const BufRsrc x_r = make_rsrc(x, xb);
        const BufRsrc u_r = make_rsrc(x + a.x2_off, silu_mul ? xb : 0);  // zero-size: loads read 0
        // The activation passes of the first 96 blocks (3072 columns) load
        // before the weights: one workgroup per CU leaves registers to spare.
        constexpr uint32_t kPass = WG / 8, kPre = (96 + kPass - 1) / kPass;
        float xv[kPre][4], uv[kPre][4];
#pragma unroll
        for (uint32_t q = 0; q < kPre; ++q) {
            if (q == 0 || q * kPass < nb) {
                x_pass_load(x_r, q * kPass, xv[q]);
                x_pass_load(u_r, q * kPass, uv[q]);
            }
        }
        // The first weight steps go out now, behind every wave's activation
        // loads (the barrier orders the issue; the CU returns
        // loads in issue order), so their HBM latency overlaps the prologue's
        // loads and the LDS fill below; the waits for the prologue data leave
        // them in flight. Activation passes beyond kPre (chunks wider than
        // 96 blocks) return behind them.
        start_chunk(nb);
        __builtin_amdgcn_s_barrier();
        issue_first();
        for (uint32_t i = threadIdx.x; i < n_tiles * 16; i += WG) row_sum[i] = 0.0f;
#pragma unroll
        for (uint32_t q = 0; q < kPre; ++q) {
            if (q == 0 || q * kPass < nb) {
                if (silu_mul) silu_mul4(xv[q], uv[q]);
                x_pass_store(xv[q], nb, q * kPass, aq, xs);
            }
        }
        for (uint32_t b0 = kPre * kPass; b0 < nb; b0 += kPass) {
            float v[4], u[4];
            x_pass_load(x_r, b0, v);
            x_pass_load(u_r, b0, u);
            if (silu_mul) silu_mul4(v, u);
            x_pass_store(v, nb, b0, aq, xs);
        }
    }
    uint32_t kb = 0;
    for (;;) {
        lds_barrier();  // activation chunk (and, first time, tables and sums) visible
        for (uint32_t j = j0; j < j1; j += kRing) {
            // Buffer q holds step j + q; the load of step j + q + DEPTH goes
            // into the buffer of step j + q - 1, computed just before.
#pragma unroll
            for (int q = 0; q < kRing; ++q) {
                if (j + q < j1) {
                    load(j + q + DEPTH < j1, nxt, rb[(q + DEPTH) % kRing], db[(q + DEPTH) % kRing]);
                    nxt = advance(nxt);
                    compute(j + q, cur, rb[q], db[q]);
                    cur = advance(cur);
                }
            }
        }
        lds_barrier();  // edge slots and whole-tile sums of this chunk written
        // Split tiles: their pieces in wave order. After the last chunk
        // thread i stores row i itself: every other contribution to it was
        // written before the barrier above.
        const bool last = kb + chunk_blk >= nblk_all;
        for (uint32_t i = threadIdx.x; i < n_tiles * 16; i += WG) {
            const uint32_t t = i >> 4, rr = i & 15;
            const uint32_t w_first = ((t * S + 1) * kWaves - 1) / L;
            const uint32_t w_last = ((t * S + S) * kWaves - 1) / L;
            float v = row_sum[i];
            if (w_first != w_last) {
                float sum = 0.0f;
                for (uint32_t w = w_first; w <= w_last; ++w) {
                    const uint32_t aw = w * L / kWaves, bw = (w + 1) * L / kWaves;
                    if (aw == bw) continue;  // empty run
                    sum += edge[aw / S == t ? 0 : 1][w * 16 + rr];
                }
                v += sum;
                if (!last) row_sum[i] = v;
            }
            if (last) {
                const uint32_t row = (t_begin + t) * 16 + rr;
                if (row < lt.rows) y_base[row] = v;
            }
        }
        if (last) break;
        kb += chunk_blk;
        // Next K-chunk (activations longer than one LDS chunk).
        const uint32_t nb = min(chunk_blk, nblk_all - kb);
        lds_barrier();  // previous chunk's LDS (activations, edge slots) no longer in use
        u_begin = kb / kBlkPerUnit;
        const uint32_t c0 = kb * 32;
        const uint32_t cb = (a.cols > c0 ? min(a.cols - c0, nb * 32) : 0) * 4;
        quantize_to_lds<WG>(make_rsrc(x + c0, cb), make_rsrc(x + a.x2_off + c0, silu_mul ? cb : 0), silu_mul, nb, aq,
                            xs);
        start_chunk(nb);
        issue_first();
    }
}

template <int UPS, int WG, int DEPTH, bool ROUTE, int NSEG>
__global__ __launch_bounds__(WG, 1024 / WG) void gemv_q_kernel(GemvSet<NSEG> set) {
    // This workgroup's segment (grid slice z).
    const GemvArgs& a = set.seg[NSEG > 1 ? blockIdx.z : 0];
    pin_gemv_args(a);
    gemv_q_body<UPS, WG, DEPTH, ROUTE, NSEG>(a, a);
}

// One segment without a problem list or silu_mul (GemvOneArgs, kernels.hpp):
// the leading scalar arguments (14 dwords) are preloaded into SGPRs.
template <int UPS, int WG, int DEPTH>
__global__ __launch_bounds__(WG, 1024 / WG) void gemv_q_one_kernel(
    const uint4* recs, const uint16_t* dvals, const float* x, uint32_t rec_stride, uint32_t d_stride, uint32_t x_stride,
    uint32_t cols, uint32_t units, uint32_t tpw_probs, uint32_t tiles, uint32_t d_row, GemvSet<1> set) {
    const GemvOneArgs a{recs,  dvals, x,     rec_stride,      d_stride,         x_stride, cols,
                        units, tpw_probs & 0xFFFFu, tiles, tpw_probs >> 16, d_row};
    gemv_q_body<UPS, WG, DEPTH, false, 1>(a, set.seg[0]);
}

// f32 / f16 weights (the router, matVecMulUnified's f32 branch): the
// reference's summation order, bit for bit. math.matVecMul (math.zig:79-99)
// keeps four accumulators, lane l summing the products of columns
// l, l + 4, l + 8, ... in column order (each product rounded, then added:
// no fused multiply-add), adds them as ((a0 + a1) + a2) + a3 (@reduce over a
// 4-vector) and then the remaining cols % 4 products one by one. f16 weights
// are widened exactly first, as dequantize does (dequant.zig:632-659).
//
// A rounded sequential sum has no parallel form, so each lane's chain runs
// in one thread. A 256-thread workgroup owns one row and NV vectors (NV > 1
// when the vectors share the matrix, as a batch of tokens shares the
// router): per chunk of kStrictChunk columns every thread forms products of
// its column quads (one load of the row's quad serves all NV vectors) and
// stores them de-interleaved, P[4v + l][i] for column 4i + l, so that chain
// (v, l) then reads four consecutive terms per LDS access and only adds.
// Products of vectors past n_vecs and columns past cols4 read as zero
// through the buffer resources and are never summed.
constexpr int kFloatThreads = 256;

template <typename WT, int NV>
__global__ __launch_bounds__(kFloatThreads) void gemv_strict_kernel(const WT* __restrict__ w, uint64_t mat_stride,
                                                                    const float* __restrict__ x, uint64_t x_stride,
                                                                    float* __restrict__ y, uint64_t y_stride,
                                                                    uint32_t n_vecs, uint32_t rows, uint32_t cols) {
#pragma clang fp contract(off)
    // Columns per product chunk (multiple of 16); a chain's row is padded by
    // four floats so the 16 chains of a lane group read disjoint banks. A
    // row of up to 2048 columns is one chunk (132 KB of LDS at NV = 16), so
    // its loads make one round trip before the chains start.
    constexpr uint32_t kStrictChunk = 2048;
    constexpr uint32_t kPRow = kStrictChunk / 4 + 4;
    __shared__ __align__(16) float P[NV * 4][kPRow];
    const uint32_t r = blockIdx.x, v0 = blockIdx.y * NV;
    const uint32_t cols4 = cols & ~3u;
    // Vector v0 + j's matrix: one shared matrix (mat_stride 0) or one each.
    const WT* wrow = w + (uint64_t)(NV == 1 ? v0 : 0) * mat_stride + (uint64_t)r * cols;
    const BufRsrc wr = make_rsrc(wrow, cols4 * (uint32_t)sizeof(WT));
    const uint32_t tid = threadIdx.x;
    // Chain thread: lanes 4v + l of wave 0 (NV <= 16).
    const uint32_t cv = tid >> 2, cl = tid & 3;
    const bool chain = tid < 4u * NV;
    float acc = 0.0f;
    for (uint32_t c0 = 0; c0 < cols4; c0 += kStrictChunk) {
        const uint32_t cn = min(kStrictChunk, cols4 - c0);
        // Product phase: column quad q = c0 / 4 + i, i = tid + 256 k.
        auto load_w = [&](uint32_t col, float (&wv)[4]) {
            if constexpr (sizeof(WT) == 2) {
                const uint2 hv = buf_load_b64(wr, col * 2, 0);
                wv[0] = f16_bits_to_f32(hv.x & 0xFFFFu);
                wv[1] = f16_bits_to_f32(hv.x >> 16);
                wv[2] = f16_bits_to_f32(hv.y & 0xFFFFu);
                wv[3] = f16_bits_to_f32(hv.y >> 16);
            } else {
                const uint4 q = buf_load_b128(wr, col * 4, 0);
                wv[0] = __uint_as_float(q.x);
                wv[1] = __uint_as_float(q.y);
                wv[2] = __uint_as_float(q.z);
                wv[3] = __uint_as_float(q.w);
            }
        };
        auto x_rsrc = [&](int j) {
            const uint32_t m = v0 + j;
            return make_rsrc(x + (uint64_t)(m < n_vecs ? m : 0) * x_stride, m < n_vecs ? cols4 * 4 : 0);
        };
        auto store = [&](uint32_t i, int j, const float (&wv)[4], const uint4& q) {
            P[4 * j + 0][i] = wv[0] * __uint_as_float(q.x);
            P[4 * j + 1][i] = wv[1] * __uint_as_float(q.y);
            P[4 * j + 2][i] = wv[2] * __uint_as_float(q.z);
            P[4 * j + 3][i] = wv[3] * __uint_as_float(q.w);
        };
        constexpr uint32_t kQpt = kStrictChunk / 4 / kFloatThreads;  // quads per thread in a full chunk
        if (NV > 1 && cn == kStrictChunk) {
            // Several vectors, full chunk: every load of the thread's quads
            // is issued before the first product, one round trip in all.
            float wv[kQpt][4];
            uint4 xq[kQpt][NV];
#pragma unroll
            for (uint32_t k = 0; k < kQpt; ++k) load_w(c0 + 4 * (tid + kFloatThreads * k), wv[k]);
#pragma unroll
            for (int j = 0; j < NV; ++j) {
                const BufRsrc xr = x_rsrc(j);
#pragma unroll
                for (uint32_t k = 0; k < kQpt; ++k) xq[k][j] = buf_load_b128(xr, (c0 + 4 * (tid + kFloatThreads * k)) * 4, 0);
            }
#pragma unroll
            for (uint32_t k = 0; k < kQpt; ++k)
#pragma unroll
                for (int j = 0; j < NV; ++j) store(tid + kFloatThreads * k, j, wv[k], xq[k][j]);
        } else {
            for (uint32_t i = tid; i < cn / 4; i += kFloatThreads) {
                const uint32_t col = c0 + 4 * i;
                float wv[4];
                load_w(col, wv);
#pragma unroll
                for (int j = 0; j < NV; ++j) store(i, j, wv, buf_load_b128(x_rsrc(j), col * 4, 0));
            }
        }
        __syncthreads();
        if (chain) {
            // The chain's terms in batches of 32 (8 x 16 bytes), read into two
            // register sets in turn so that the next batch's LDS reads are in
            // flight while the current one is added (the adds are one
            // dependent sequence; only the read latency can be hidden). The
            // read after the last batch re-reads it (clamped) and is unused.
            // One vector (a decode router): the chain is the whole row and
            // its read latency shows. Several vectors: 4 NV chains per
            // workgroup overlap each other's reads, and the two register
            // sets measured slower (7.1 -> 12.1 us for 64 tokens).
            const float4* pp = reinterpret_cast<const float4*>(&P[tid][0]);
            const uint32_t n16 = cn / 16, nb = NV == 1 ? n16 / 8 : 0;
            float4 ra[8], rb[8];
            auto read = [&](float4 (&r)[8], uint32_t b) {
#pragma unroll
                for (int k = 0; k < 8; ++k) r[k] = pp[b * 8 + k];
                // Keeps the reads issued here, ahead of the adds that follow.
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
            // cn is a multiple of 4 but not always of 16: the last quad-steps.
            for (uint32_t i = n16 * 4; i < cn / 4; ++i) acc = acc + P[tid][i];
        }
        __syncthreads();
    }
    // ((a0 + a1) + a2) + a3 in lane l = 0 of each chain, then the tail.
    const float a1 = __shfl_down(acc, 1, kWave), a2 = __shfl_down(acc, 2, kWave), a3 = __shfl_down(acc, 3, kWave);
    if (chain && cl == 0 && v0 + cv < n_vecs) {
        const uint32_t m = v0 + cv;
        float sum = ((acc + a1) + a2) + a3;
        const WT* wm = w + (uint64_t)(NV == 1 ? m : 0) * mat_stride + (uint64_t)r * cols;
        const float* xm = x + (uint64_t)m * x_stride;
        for (uint32_t j = cols4; j < cols; ++j) {
            float wj;
            if constexpr (sizeof(WT) == 2)
                wj = f16_bits_to_f32(wm[j]);
            else
                wj = wm[j];
            sum = sum + wj * xm[j];
        }
        y[(uint64_t)m * y_stride + r] = sum;
    }
}

}  // namespace

static size_t gemv_q_lds_bytes(uint32_t units) {
    const uint32_t nblk = units * 2;
    const uint32_t chunk = nblk < kChunkBlocks ? nblk : kChunkBlocks;
    return (size_t)((chunk + 7) / 8) * kAGroupBytes + (size_t)chunk * 4;
}

// Units per step: a divisor of both the tile's unit count and the LDS
// chunk's. Q8_0 tiles hold a multiple of 4 units (256-column A groups), and
// steps are 4 or 8 units.
static int pick_ups(uint32_t units) {
    const uint32_t chunk_units = min(units, (uint32_t)(kChunkBlocks / 2));
    uint32_t a = units, b = chunk_units;
    while (b) {
        const uint32_t t = a % b;
        a = b;
        b = t;
    }
    const uint32_t common = a;
    if (common % 8 == 0) return 8;
    if (common % 4 == 0) return 4;
    return 0;
}

template <int WG, int DEPTH, bool ROUTE, int NSEG>
static const void* kernel_for(int ups) {
    return ups == 8 ? reinterpret_cast<const void*>(&gemv_q_kernel<8, WG, DEPTH, ROUTE, NSEG>)
                    : reinterpret_cast<const void*>(&gemv_q_kernel<4, WG, DEPTH, ROUTE, NSEG>);
}

static int env_int(const char* name, int dflt) {
    const char* e = getenv(name);
    return e ? atoi(e) : dflt;
}

template <int DEPTH>
static const void* kernel_for_wg(int wg, int ups) {
    if (wg == 1024) return kernel_for<1024, DEPTH, false, 1>(ups);
    return kernel_for<256, DEPTH, false, 1>(ups);
}

template <int DEPTH>
static const void* one_kernel_for(int wg, int ups) {
    if (wg == 1024)
        return ups == 8 ? reinterpret_cast<const void*>(&gemv_q_one_kernel<8, 1024, DEPTH>)
                        : reinterpret_cast<const void*>(&gemv_q_one_kernel<4, 1024, DEPTH>);
    return ups == 8 ? reinterpret_cast<const void*>(&gemv_q_one_kernel<8, 256, DEPTH>)
                    : reinterpret_cast<const void*>(&gemv_q_one_kernel<4, 256, DEPTH>);
}

template <int N>
static hipError_t launch_q_set(const GemvArgs* segs, uint32_t n_segs, const void* fn, uint32_t grid_x, int wg,
                               size_t lds, hipStream_t s) {
    GemvSet<N> set{};
    uint32_t y = 0;
    for (uint32_t i = 0; i < (uint32_t)N; ++i) {
        set.seg[i] = segs[i < n_segs ? i : 0];
        if (i < n_segs && segs[i].n_probs > y) y = segs[i].n_probs;
    }
    void* args[] = {&set};
    return hipLaunchKernel(fn, dim3(grid_x, y, n_segs), dim3(wg), args, lds, s);
}

hipError_t launch_gemv_q(const GemvArgs& a, uint32_t fmt, int num_cu, hipStream_t s) {
    return launch_gemv_segments(&a, 1, fmt, num_cu, s);
}

hipError_t launch_gemv_segments(const GemvArgs* segs_in, uint32_t n_segs, uint32_t fmt, int num_cu, hipStream_t s) {
    if (n_segs == 0 || n_segs > kGemvMaxSegs) return hipErrorInvalidValue;
    if (fmt == kFmtIq2) return launch_gemv_iq2(segs_in, n_segs, num_cu, s);
    GemvArgs segs[kGemvMaxSegs];
    uint32_t n = 0;
    for (uint32_t i = 0; i < n_segs; ++i)
        if (segs_in[i].n_probs && segs_in[i].tiles) segs[n++] = segs_in[i];
    if (n == 0) return hipSuccess;
    const bool route = segs[0].route_decode != 0;
    if (route && n != 1) return hipErrorInvalidValue;
    // Defaults measured on MI355X with 64-matrix batches: 256 threads, one
    // workgroup per CU, two steps of 4 units in flight: four long streams
    // per CU keep fewer requests outstanding and reach a higher HBM rate than
    // sixteen. Overrides: MMHIP_GEMV_WG (256 | 1024), MMHIP_GEMV_MAX_UPS (4 |
    // 8 record units per step), MMHIP_GEMV_DEPTH (steps in flight, 1..3;
    // default below).
    static const int wg_env = env_int("MMHIP_GEMV_WG", 0);
    static const int cap_env = env_int("MMHIP_GEMV_MAX_UPS", 0);
    static const int depth_env = env_int("MMHIP_GEMV_DEPTH", 0);
    const int wg = wg_env == 1024 && n == 1 ? 1024 : 256;
    // Steps above 4 units exceed the register budget with two record
    // buffers in flight and spill. A step size must divide every segment's
    // tile and chunk unit counts.
    const int cap = cap_env == 8 ? 8 : 4;
    int ups = cap;
    size_t lds = 0;
    for (uint32_t i = 0; i < n; ++i) {
        int u = pick_ups(segs[i].units);
        if (u == 0) return hipErrorInvalidValue;
        if (u < ups) ups = u;
        const size_t l = gemv_q_lds_bytes(segs[i].units);
        if (l > lds) lds = l;
    }
    // Tiles per workgroup: the problems' tiles spread over one workgroup per
    // CU (several segments: about the same record units per workgroup), at
    // most kGemvMaxTiles (the LDS row sums).
    const uint64_t target_wgs = (uint64_t)(num_cu > 0 ? num_cu : 256);
    uint32_t grid_x = 1;
    if (n == 1) {
        GemvArgs& a = segs[0];
        uint64_t tpw = ((uint64_t)a.n_probs * a.tiles + target_wgs - 1) / target_wgs;
        if (tpw > kGemvMaxTiles) tpw = kGemvMaxTiles;
        if (tpw > a.tiles) tpw = a.tiles;
        a.tiles_per_wg = (uint32_t)tpw;
        grid_x = (a.tiles + a.tiles_per_wg - 1) / a.tiles_per_wg;
    } else {
        uint64_t units = 0;
        for (uint32_t i = 0; i < n; ++i) units += (uint64_t)segs[i].n_probs * segs[i].tiles * segs[i].units;
        const uint64_t per_wg = (units + target_wgs - 1) / target_wgs;
        for (uint32_t i = 0; i < n; ++i) {
            GemvArgs& a = segs[i];
            uint64_t t = (per_wg + a.units - 1) / a.units;
            if (t > kGemvMaxTiles) t = kGemvMaxTiles;
            if (t > a.tiles) t = a.tiles;
            if (t < 1) t = 1;
            a.tiles_per_wg = (uint32_t)t;
            const uint32_t gx = (a.tiles + a.tiles_per_wg - 1) / a.tiles_per_wg;
            if (gx > grid_x) grid_x = gx;
        }
    }
    // One step in flight when every workgroup has a single tile and each
    // wave at most two steps (one matrix of at most a tile per CU: a
    // [1536 x 2048] call, most MLA projections): both steps then go out at
    // the start, and a deeper ring would only add out-of-range loads to the
    // queue (MLA Q8_0 decode 19.9 -> 19.2 us per layer). Waves with three or
    // more steps, and larger launches (HBM-bound), keep two.
    const uint32_t chunk_steps = (min(segs[0].units, kChunkBlocks / 2) + ups - 1) / ups;
    const bool short_waves = n == 1 && segs[0].tiles_per_wg == 1 && chunk_steps <= 2 * (uint32_t)(wg / 64);
    const int depth = (depth_env >= 1 && depth_env <= 3) ? depth_env : (short_waves ? 1 : 2);
    if (route) return launch_q_set<1>(segs, 1, kernel_for<256, 2, true, 1>(ups), grid_x, 256, lds, s);
    if (n == 1) {
        const GemvArgs& a = segs[0];
        if (!a.probs && !a.n_active && !a.silu_mul && a.rec_stride < (1ull << 27) && a.d_stride < (1ull << 30) &&
            a.x_stride < (1ull << 32) && a.n_probs < 65536 && a.tiles_per_wg < 65536) {
            // Preloaded arguments (gemv_q_one_kernel).
            const void* fn = depth == 1   ? one_kernel_for<1>(wg, ups)
                             : depth == 3 ? one_kernel_for<3>(wg, ups)
                                          : one_kernel_for<2>(wg, ups);
            GemvSet<1> set{};
            set.seg[0] = a;
            const uint4* recs = a.recs + a.first_mat * a.rec_stride;
            const uint16_t* dvals = a.dvals + a.first_mat * a.d_stride;
            const float* x = a.x;
            uint32_t rs = (uint32_t)a.rec_stride, ds = (uint32_t)a.d_stride, xs = (uint32_t)a.x_stride;
            uint32_t cols = a.cols, units = a.units, tpw_np = a.tiles_per_wg | (a.n_probs << 16), tiles = a.tiles,
                     drow = a.d_row;
            void* args[] = {&recs, &dvals, &x, &rs, &ds, &xs, &cols, &units, &tpw_np, &tiles, &drow, &set};
            return hipLaunchKernel(fn, dim3(grid_x, a.n_probs, 1), dim3(wg), args, lds, s);
        }
        const void* fn =
            depth == 1 ? kernel_for_wg<1>(wg, ups) : depth == 3 ? kernel_for_wg<3>(wg, ups) : kernel_for_wg<2>(wg, ups);
        return launch_q_set<1>(segs, 1, fn, grid_x, wg, lds, s);
    }
    if (n == 2) return launch_q_set<2>(segs, 2, kernel_for<256, 2, false, 2>(ups), grid_x, 256, lds, s);
    return launch_q_set<4>(segs, n, kernel_for<256, 2, false, 4>(ups), grid_x, 256, lds, s);
}

hipError_t launch_gemv_float(const void* w, uint32_t type, uint64_t mat_stride, const float* x,
                             uint64_t x_stride, float* y, uint64_t y_stride, uint32_t n_mats,
                             uint32_t rows, uint32_t cols, hipStream_t s) {
    if ((uint64_t)n_mats * rows == 0) return hipSuccess;
    if (mat_stride == 0 && n_mats > 1) {
        // One matrix, several vectors: 16 vectors per workgroup.
        const dim3 grid(rows, (n_mats + 15) / 16);
        if (type == 0)
            gemv_strict_kernel<float, 16><<<grid, kFloatThreads, 0, s>>>((const float*)w, 0, x, x_stride, y, y_stride,
                                                                         n_mats, rows, cols);
        else
            gemv_strict_kernel<uint16_t, 16><<<grid, kFloatThreads, 0, s>>>((const uint16_t*)w, 0, x, x_stride, y,
                                                                            y_stride, n_mats, rows, cols);
        return hipGetLastError();
    }
    const dim3 grid(rows, n_mats);
    if (type == 0)
        gemv_strict_kernel<float, 1><<<grid, kFloatThreads, 0, s>>>((const float*)w, mat_stride, x, x_stride, y,
                                                                    y_stride, n_mats, rows, cols);
    else
        gemv_strict_kernel<uint16_t, 1><<<grid, kFloatThreads, 0, s>>>((const uint16_t*)w, mat_stride, x, x_stride, y,
                                                                       y_stride, n_mats, rows, cols);
    return hipGetLastError();
}

}  // namespace mmhip
