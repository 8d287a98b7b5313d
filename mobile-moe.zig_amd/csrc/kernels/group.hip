// Quantised matmul over groups of 8 activation rows on gfx950: prompt prefill
// (qmm.matMulQ8_0's role, qmm.zig:58-138) and the MoE experts of a batch
// grouped by expert (moeFFN over forwardBatch's tokens, inference.zig:346-351,
// 886-1188).
//
// An item is one weight matrix and up to 8 activation rows: consecutive rows
// of a batch (dense) or the slots of one expert (grouped, items written by the
// route kernel). The activations arrive quantised (two int8 digit planes +
// per-block scales) and are staged into LDS so that row j's digits are the A
// rows 2j / 2j+1 of v_mfma_i32_16x16x32_i8: all 16 A rows carry data, and each
// weight unit's B operands (IQ2_XXS table lookups or raw Q8_0 bytes) are built
// once for 8 rows. Lane (n, g) ends with rows 2g and 2g+1 of weight row n; no
// cross-lane reduction is needed.
//
// Streaming is the decode GEMV's: unconditional buffer loads, a ring of three
// register buffers, an LDS-only barrier, tables copied into LDS.
#include "device_common.hpp"
#include "kernels.hpp"
#include "tile_ops.hpp"

#include <cstdlib>
#include <map>
#include <mutex>

namespace mmhip {

namespace {

constexpr uint32_t kGRows = 8;            // activation rows per item
constexpr uint32_t kGChunkBlocks = 64;    // 2048 columns of activations per LDS chunk
constexpr uint32_t kGStage = kGChunkBlocks / 2 * 64;  // 16-byte A chunks per LDS chunk

struct GroupArgs {
    const uint4* recs;
    const uint16_t* dvals;
    uint64_t rec_stride, d_stride;
    uint32_t d_row;
    const int8_t* xh;
    const int8_t* xl;
    const float* xs;
    uint64_t xq_stride, xs_stride;
    const uint32_t* a_row;          // slot -> activation row (grouped), or null
    float* y;
    uint64_t y_slot, y_row;         // y[slot * y_slot + col_off + row * y_row]
    const QmmWork* work;            // grouped when non-null
    const uint32_t* n_work;
    uint64_t mat;                   // dense: matrix
    uint32_t batch;                 // dense: rows of the batch
    uint32_t tiles, units, rows;
    uint32_t gap;                   // grouped: tiles of range an item boundary counts for (see below)
};

// LDS A layout of one chunk: block pair p (blocks 2p, 2p+1) is 1 KiB; lane
// (n, g)'s 16 bytes at p * 1024 + lane * 16 hold A row n (activation row n/2,
// digit n&1), columns 8g..8g+7 of block 2p, then of block 2p+1. Lanes read
// consecutive 16-byte words: no bank conflicts.
__device__ __forceinline__ void lds_a_pair(const uint8_t* aq, uint32_t pair, uint32_t lane, long& a0, long& a1) {
    const uint4 q = *reinterpret_cast<const uint4*>(aq + pair * 1024 + lane * 16);
    a0 = (long)(((uint64_t)q.y << 32) | q.x);
    a1 = (long)(((uint64_t)q.w << 32) | q.z);
}

// One step of UPS IQ2_XXS units (unit u = 256 columns = 4 block pairs) for 8
// activation rows; xs_lds[j * nb + b] = scale of row j, block b of the chunk.
// The activations carry one scale per unit (quantised wide), so a unit's
// value for row n and activation row j is
//   d_n / 8 * s_j * sum_s (2 ls_ns + 1) * (256 D_hi,s + D_lo,s)
// (dequant.zig:336: d * (0.5 + ls) / 4): the eight blocks' digit dot products
// are weighted by 2 ls + 1 and summed exactly in int32 (24-bit multiplies:
// |D| <= 32 * 128 * 43, weighted sums < 2^26), then converted and scaled once.
// B operands of one IQ2_XXS record unit with every LDS read (8 record
// entries, 8 hi3 mask pairs) issued before the first sign fix, so the unit
// waits for the table once instead of once per batch of reads; the same
// values as iq2_decode_unit.
__device__ __forceinline__ void iq2_decode_unit_batched(const uint4& rr, const uint32_t* tab, long (&b)[8]) {
    const uint32_t w4[4] = {rr.x, rr.y, rr.z, rr.w};
    const char* t8 = reinterpret_cast<const char*>(tab);
    const char* m8 = t8 + kIq2TableWords * 4;
    uint2 e[8], m[8];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t d = w4[k];
        e[2 * k] = *reinterpret_cast<const uint2*>(t8 + (d & 0x7FF8u));
        m[2 * k] = *reinterpret_cast<const uint2*>(m8 + ((d >> 12) & 0x38u));
        e[2 * k + 1] = *reinterpret_cast<const uint2*>(t8 + ((d >> 15) & 0x7FF8u));
        m[2 * k + 1] = *reinterpret_cast<const uint2*>(m8 + ((d << 3) & 0x38u));
    }
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        // (e.y ^ m.x) + m.y as one v_xad_u32 (as plain C the compiler
        // folds the add into a 64-bit add with the low word: three VALU).
        uint32_t hi;
        asm("v_xad_u32 %0, %1, %2, %3" : "=v"(hi) : "v"(e[s].y), "v"(m[s].x), "v"(m[s].y));
        b[s] = __builtin_bit_cast(long, make_uint2(e[s].x, hi));
    }
}

template <int UPS>
__device__ __forceinline__ void step_group_iq2(const uint4 (&r)[kMaxUnitsPerStep], const uint32_t (&dw)[kMaxUnitsPerStep],
                                               uint32_t ub, const uint8_t* aq, const float* xs0, const float* xs1,
                                               const uint32_t* tab, uint32_t lane, float& acc0, float& acc1) {
    const uint32_t g = lane >> 4;
    long b[2][8];
    long av[8];
    // The first unit's activation reads go out before its table reads, so
    // both arrive in one LDS round trip.
#pragma unroll
    for (int q = 0; q < 4; ++q) lds_a_pair(aq, ub * 4 + q, lane, av[2 * q], av[2 * q + 1]);
    iq2_decode_unit_batched(r[0], tab, b[0]);
#pragma unroll
    for (int i = 0; i < UPS; ++i) {
        const int cur = i & 1, nxt = cur ^ 1;
        if (i > 0) {
#pragma unroll
            for (int q = 0; q < 4; ++q) lds_a_pair(aq, (ub + i) * 4 + q, lane, av[2 * q], av[2 * q + 1]);
        }
        const uint32_t blk0 = (ub + i) * 8;
        const float x0 = xs0[blk0], x1 = xs1[blk0];
        const uint32_t ls = iq2_ls_all(r[i], g);
        if (i + 1 < UPS) iq2_decode_unit_batched(r[i + 1], tab, b[nxt]);
        int h0 = 0, l0 = 0, h1 = 0, l1 = 0;
        // Block s's MFMA is issued before block s - 1's products are
        // weighted, so each MFMA's latency overlaps the previous block's
        // multiply-adds instead of stalling the wave (the sums are integer:
        // the order of the adds does not change them).
        v4i dv[2];
        dv[0] = mfma_i8(av[0], b[cur][0]);
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            if (s + 1 < 8) dv[(s + 1) & 1] = mfma_i8(av[s + 1], b[cur][s + 1]);
            const v4i& d = dv[s & 1];
            const int t = (int)(((ls >> (4 * s)) & 15u) * 2 + 1);
            h0 = __mul24(d[0], t) + h0;
            l0 = __mul24(d[1], t) + l0;
            h1 = __mul24(d[2], t) + h1;
            l1 = __mul24(d[3], t) + l1;
            // Keeps each sum a chain of 24-bit multiply-adds (one
            // instruction per product) instead of products plus add trees.
            asm("" : "+v"(h0), "+v"(l0), "+v"(h1), "+v"(l1));
        }
        const float c = f16_scale(iq2_scale_bits<UPS>(dw, i)) * 0.125f;
        acc0 = fmaf(fmaf((float)h0, 256.0f, (float)l0), c * x0, acc0);
        acc1 = fmaf(fmaf((float)h1, 256.0f, (float)l1), c * x1, acc1);
    }
}

// Q8_0: unit u = 64 columns = block pair u.
template <int UPS>
__device__ __forceinline__ void step_group_q8(const uint4 (&r)[kMaxUnitsPerStep], const uint32_t (&dw)[kMaxUnitsPerStep],
                                              uint32_t ub, const uint8_t* aq, const float* xs0, const float* xs1,
                                              uint32_t lane, float& acc0, float& acc1) {
#pragma unroll
    for (int i = 0; i < UPS; ++i) {
        long a0, a1;
        lds_a_pair(aq, ub + i, lane, a0, a1);
        const uint32_t blk0 = (ub + i) * 2;
        const float2 x0 = *reinterpret_cast<const float2*>(xs0 + blk0);
        const float2 x1 = *reinterpret_cast<const float2*>(xs1 + blk0);
        const uint4& rr = r[i];
        const v4i d0 = mfma_i8(a0, (long)(((uint64_t)rr.y << 32) | rr.x));
        const v4i d1 = mfma_i8(a1, (long)(((uint64_t)rr.w << 32) | rr.z));
        const float w0 = f16_scale(dw[i] & 0xFFFFu), w1 = f16_scale(dw[i] >> 16);
        acc0 = fmaf((float)digits_combine(d0[0], d0[1]), w0 * x0.x, acc0);
        acc1 = fmaf((float)digits_combine(d0[2], d0[3]), w0 * x1.x, acc1);
        acc0 = fmaf((float)digits_combine(d1[0], d1[1]), w1 * x0.y, acc0);
        acc1 = fmaf((float)digits_combine(d1[2], d1[3]), w1 * x1.y, acc1);
    }
}

// The launch bound's second argument is the minimum waves per SIMD: two
// 512-thread IQ2_XXS workgroups share a CU (their LDS fits twice), or one
// 1024-thread workgroup fills it: four waves per SIMD either way, so at most
// 128 registers.
template <int FMT, int UPS, int WG>
__global__ __launch_bounds__(WG, (FMT == kFmtIq2 && WG >= 512) ? 4 : 2) void group_kernel(GroupArgs a) {
    constexpr uint32_t kWaves = WG / 64;
    constexpr uint32_t kBlkPerUnit = (FMT == kFmtIq2) ? 8 : 2;
    __shared__ __align__(16) uint32_t tab[FMT == kFmtIq2 ? kIq2LdsWords : 4];
    __shared__ __align__(16) uint8_t aq[kGChunkBlocks * 512];
    __shared__ __align__(16) float xs_lds[kGRows * kGChunkBlocks];

    // This workgroup's share of the (item, row tile) pairs, item-major:
    // equal contiguous ranges over the grid, so every workgroup streams the
    // same number of tiles whatever number of items the routing produced
    // (the host sizes the grid before the routing runs). A range covers whole
    // or partial tile runs of one or two items; the activations are staged
    // once per item run.
    //
    // Grouped 1024-thread launches (a.gap > 0; the host sets it): a range
    // that crosses into a new item pays for the switch (the pipeline
    // drains, then the item's work entry, rows, digits and first weights come
    // in series: ~5.5 steps per wave, s_memrealtime per workgroup), and the
    // workgroups that cross set the launch's end. So the ranges are cut
    // equally on a line where every item counts a.gap extra tiles after its
    // own: a crossing workgroup gets about a switch's worth fewer tiles.
    // Position v of that line is item v / vlen, tile min(v % vlen, tiles): the
    // map is monotone and onto, so the ranges still cover every (item, tile)
    // exactly once.
    const uint32_t n_items = a.work ? *a.n_work : (a.batch + kGRows - 1) / kGRows;
    const uint64_t vlen = (uint64_t)a.tiles + a.gap;
    const uint64_t total_v = (uint64_t)n_items * vlen;
    auto real_pos = [&](uint64_t v) {
        const uint64_t it = v / vlen, off = v % vlen;
        return it * a.tiles + (off < a.tiles ? off : a.tiles);
    };
    uint64_t q = real_pos(total_v * blockIdx.x / gridDim.x);
    const uint64_t q_end = real_pos(total_v * (blockIdx.x + 1) / gridDim.x);
    if (q >= q_end) return;  // whole workgroup

    const uint32_t lane = threadIdx.x & 63;
    const uint32_t n = lane & 15, g = lane >> 4;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t nblk_all = a.units * kBlkPerUnit;
    const uint32_t chunk_blk = nblk_all < kGChunkBlocks ? nblk_all : kGChunkBlocks;
    const uint32_t chunk_units = chunk_blk / kBlkPerUnit;
    const uint32_t rec_voff = lane * 16;
    const uint32_t d_voff = n * a.d_row * 2;

    // Current item run: matrix, first slot, rows, output column offset, and
    // tiles [t_begin, t_begin + run) split over the waves (wave v: t_begin +
    // v + kWaves i).
    uint64_t mat = a.mat;
    uint32_t first = 0, count = 0, col_off = 0, t_begin = 0, my_n = 0;
    BufRsrc rec_r = make_rsrc(a.recs, 0u), d_r = make_rsrc(a.dvals, 0u);  // set by next_run
    // Activation row of item row j (rows past `count` repeat row 0: their
    // results are computed and dropped).
    auto act_row = [&](uint32_t j) -> uint64_t {
        const uint32_t s = first + (j < count ? j : 0);
        return (a.work && a.a_row) ? a.a_row[s] : s;
    };

    uint32_t u_begin = 0;
    uint32_t n_sub = 1, steps = 0;
    auto tile_of = [&](uint32_t s) { return t_begin + wave + kWaves * (s / n_sub); };
    auto first_unit = [&](uint32_t s) { return u_begin + (s % n_sub) * UPS; };
    uint4 r0[kMaxUnitsPerStep], r1[kMaxUnitsPerStep], r2[kMaxUnitsPerStep];
    uint32_t d0[kMaxUnitsPerStep], d1[kMaxUnitsPerStep], d2[kMaxUnitsPerStep];
    auto load = [&](uint32_t s, uint4 (&r)[kMaxUnitsPerStep], uint32_t (&dw)[kMaxUnitsPerStep]) {
        uint32_t rs = kBufOob, ds = kBufOob;
        if (s < steps) {
            const uint32_t t = tile_of(s), u = first_unit(s);
            rs = (t * a.units + u) * 1024;
            ds = (t * 16 * a.d_row + u * (FMT == kFmtIq2 ? 1 : 2)) * 2;
        }
        load_step<FMT, UPS>(rec_r, rec_voff, rs, d_r, d_voff, ds, r, dw);
    };
    float acc0 = 0.0f, acc1 = 0.0f;
    uint32_t kb = 0;
    const float* xs0 = xs_lds + (2 * g) * kGChunkBlocks;
    const float* xs1 = xs0 + kGChunkBlocks;
    auto compute = [&](uint32_t s, const uint4 (&r)[kMaxUnitsPerStep], const uint32_t (&dw)[kMaxUnitsPerStep]) {
        const uint32_t ub = first_unit(s) - u_begin;
        if (FMT == kFmtIq2)
            step_group_iq2<UPS>(r, dw, ub, aq, xs0, xs1, tab, lane, acc0, acc1);
        else
            step_group_q8<UPS>(r, dw, ub, aq, xs0, xs1, lane, acc0, acc1);
        if (s % n_sub == n_sub - 1) {
            const uint32_t row = tile_of(s) * 16 + n;
            if (row < a.rows) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const uint32_t j = 2 * g + h;
                    if (j < count) {
                        float* yp = a.y + (uint64_t)(first + j) * a.y_slot + col_off + (uint64_t)row * a.y_row;
                        const float v = h ? acc1 : acc0;
                        *yp = (kb == 0) ? v : *yp + v;
                    }
                }
            }
            acc0 = acc1 = 0.0f;
        }
    };
    // Stage chunk [kb, kb + nb) of the item's activations: thread t moves the
    // 16-byte A words c = t + i * WG (all of activation row ((t & 15) >> 1),
    // WG being a multiple of 16) and the scales (j, b) = t + i * WG.
    constexpr uint32_t kPer = kGStage / WG;
    constexpr uint32_t kScales = kGRows * kGChunkBlocks;
    constexpr uint32_t kPerSc = (kScales + WG - 1) / WG;
    static_assert(WG % 16 == 0, "a thread's A words share one activation row");
    // This thread's activation rows in the current run, read once per run by
    // load_rows (next_run), before the run's other loads: read inside the
    // staging loop, each row's load and the wait for it came after the
    // table and earlier staging loads, and vector loads return in issue
    // order, so every iteration waited for all of them.
    uint64_t xrow = 0, srow[kPerSc];
    auto load_rows = [&]() {
        xrow = act_row((threadIdx.x & 15) >> 1);
#pragma unroll
        for (uint32_t i = 0; i < kPerSc; ++i) {
            const uint32_t e = threadIdx.x + i * WG;
            srow[i] = act_row((e < kScales ? e : 0) / kGChunkBlocks);
        }
    };
    auto stage_load = [&](uint32_t kb0, uint32_t nb, uint2 (&lo)[kPer], uint2 (&hi)[kPer], float (&sc)[kPerSc]) {
        const int8_t* plane = (threadIdx.x & 1) ? a.xl : a.xh;
#pragma unroll
        for (uint32_t i = 0; i < kPer; ++i) {
            const uint32_t c = threadIdx.x + i * WG;
            const uint32_t p = c >> 6, l = c & 63, lg = l >> 4;
            const bool ok = 2 * p < nb;
            const int8_t* src = plane + xrow * a.xq_stride + (kb0 + 2 * (ok ? p : 0)) * 32 + 8 * lg;
            lo[i] = *reinterpret_cast<const uint2*>(src);
            hi[i] = *reinterpret_cast<const uint2*>(src + 32);
        }
#pragma unroll
        for (uint32_t i = 0; i < kPerSc; ++i) {
            const uint32_t e = threadIdx.x + i * WG;
            const uint32_t b = e % kGChunkBlocks;
            sc[i] = a.xs[srow[i] * a.xs_stride + kb0 + (b < nb ? b : 0)];
        }
    };
    auto stage_store = [&](uint32_t nb, const uint2 (&lo)[kPer], const uint2 (&hi)[kPer], const float (&sc)[kPerSc]) {
#pragma unroll
        for (uint32_t i = 0; i < kPer; ++i) {
            const uint32_t c = threadIdx.x + i * WG;
            if (2 * (c >> 6) < nb) *reinterpret_cast<uint4*>(aq + c * 16) = make_uint4(lo[i].x, lo[i].y, hi[i].x, hi[i].y);
        }
#pragma unroll
        for (uint32_t i = 0; i < kPerSc; ++i) {
            const uint32_t e = threadIdx.x + i * WG;
            if (e < kScales && e % kGChunkBlocks < nb) xs_lds[e] = sc[i];
        }
    };

    // Takes the next run of the range: its item and tiles.
    auto next_run = [&]() {
        const uint32_t item = (uint32_t)(q / a.tiles);
        t_begin = (uint32_t)(q % a.tiles);
        const uint32_t run = (uint32_t)min((uint64_t)(a.tiles - t_begin), q_end - q);
        q += run;
        if (a.work) {
            const QmmWork w = a.work[item];
            mat = w.mat;
            first = w.slot;
            count = w.count;
            col_off = w.pad;
        } else {
            first = item * kGRows;
            count = min(a.batch - first, kGRows);
        }
        my_n = wave < run ? (run - wave + kWaves - 1) / kWaves : 0;
        rec_r = make_rsrc(a.recs + mat * a.rec_stride, (uint32_t)(a.rec_stride * 16));
        d_r = make_rsrc(a.dvals + mat * a.d_stride, (uint32_t)(a.d_stride * 2));
        u_begin = 0;
        n_sub = min(a.units, chunk_units) / UPS;
        steps = my_n * n_sub;
        kb = 0;
        load_rows();
    };
    next_run();
    {
        // Small loads first: a CU returns loads in issue order across its
        // waves, so weights issued earlier would hold them back. Every wave's
        // small loads are issued (barrier) before the first weight loads go
        // out; their latencies then overlap, and the LDS stores below wait
        // only for the small loads.
        Iq2TableCopy<WG> tc;
        if (FMT == kFmtIq2) tc.load();
        uint2 lo[kPer], hi[kPer];
        float sc[kPerSc];
        stage_load(0, chunk_blk, lo, hi, sc);
        __builtin_amdgcn_s_barrier();
        load(0, r0, d0);
        load(1, r1, d1);
        load(2, r2, d2);
        if (FMT == kFmtIq2) tc.store(tab);
        stage_store(chunk_blk, lo, hi, sc);
    }
    for (;;) {
        lds_barrier();
        for (uint32_t s = 0; s < steps; s += 3) {
            if constexpr (WG == 1024) {
                // Issue priority by steps left (a SIMD serves its oldest wave
                // first; the youngest would otherwise end last).
                const uint32_t rem = steps - s;
                if (rem > 12) __builtin_amdgcn_s_setprio(3);
                else if (rem > 6) __builtin_amdgcn_s_setprio(2);
                else if (rem > 3) __builtin_amdgcn_s_setprio(1);
                else __builtin_amdgcn_s_setprio(0);
            }
            compute(s, r0, d0);
            load(s + 3, r0, d0);
            if (s + 1 < steps) compute(s + 1, r1, d1);
            load(s + 4, r1, d1);
            if (s + 2 < steps) compute(s + 2, r2, d2);
            load(s + 5, r2, d2);
        }
        kb += chunk_blk;
        uint32_t kb0 = kb, nb = chunk_blk;
        if (kb < nblk_all) {
            // Next K-chunk of this run.
            nb = min(chunk_blk, nblk_all - kb);
            u_begin = kb / kBlkPerUnit;
            n_sub = (nb / kBlkPerUnit) / UPS;
            steps = my_n * n_sub;
        } else {
            if (q >= q_end) break;
            next_run();  // the next item's run, from its first chunk
            kb0 = 0;
        }
        lds_barrier();  // the previous chunk's LDS no longer in use
        uint2 lo[kPer], hi[kPer];
        float sc[kPerSc];
        stage_load(kb0, nb, lo, hi, sc);
        if (kb0 == 0) __builtin_amdgcn_s_barrier();  // a new item: every wave's small loads ahead of its weights
        load(0, r0, d0);
        load(1, r1, d1);
        load(2, r2, d2);
        stage_store(nb, lo, hi, sc);
    }
}

// Dense Q8_0 matmul for K <= 2048 with the activation quantisation fused in
// and each tile's K range split over KS waves. A workgroup is one item (8
// activation rows) and 16 / KS row tiles; wave (ts, ks) streams units
// [ks * units / KS, (ks + 1) * units / KS) of tile ts (one or two steps of
// four units), all issued before the first product, so a wave waits for its
// weights once. The workgroup quantises its item's rows straight into the
// LDS A layout (quantize_quad: the digits and scales quantize_kernel
// writes), so the call is one launch. Partial sums of a tile are added in
// slice order (ks = 0, 1, ..) by its first wave.
struct QmmQ8Args {
    const uint4* recs;
    const uint16_t* dvals;
    uint64_t rec_stride, d_stride;
    uint32_t d_row;
    const float* x;
    uint32_t x_stride;              // floats between rows
    uint32_t x_bytes;               // batch rows of x (< 2^31)
    uint32_t cols;                  // columns of x read (a multiple of 32; past them: zeros)
    float* y;
    uint64_t y_slot, y_row;         // y[b * y_slot + r * y_row]
    uint64_t mat;
    uint32_t batch, tiles, units, rows;
    uint32_t tgroups;               // ceil(tiles / (16 / KS))
};

template <int KS>
__global__ __launch_bounds__((16 / KS) * KS * 64) void qmm_q8_fused_kernel(QmmQ8Args a) {
    constexpr int UPS = 4;  // Q8_0 steps load their scales as 16-byte words
    constexpr uint32_t kTpw = 16 / KS;      // tiles per workgroup
    constexpr uint32_t kWaves = kTpw * KS;  // 14..16
    constexpr uint32_t kPasses = (kGChunkBlocks + kWaves - 1) / kWaves;
    __shared__ __align__(16) uint8_t aq[kGChunkBlocks * 512];
    __shared__ __align__(16) float xs_lds[kGRows * kGChunkBlocks];
    __shared__ float red[KS > 1 ? kTpw * (KS - 1) * 2 * 64 : 1];

    // Block b -> (item, tile group): the eight workgroups b = 8 r + x (one
    // per XCD) take tile groups 8 (r / items) + x of item r % items, so each
    // XCD's L2 holds one eighth of the matrix for every item.
    // Every argument read at once (one batch of scalar loads, one wait;
    // read where first used, the early exit below waited for its own loads
    // first: a second kernel-argument round trip).
    asm volatile("" ::"s"(a.recs), "s"(a.dvals), "s"(a.rec_stride), "s"(a.d_stride), "s"(a.d_row), "s"(a.x),
                 "s"(a.x_stride), "s"(a.x_bytes), "s"(a.cols), "s"(a.y), "s"(a.y_slot), "s"(a.y_row), "s"(a.mat),
                 "s"(a.batch), "s"(a.tiles), "s"(a.units), "s"(a.rows), "s"(a.tgroups));
    const uint32_t n_items = (a.batch + kGRows - 1) / kGRows;
    const uint32_t xcd = blockIdx.x & 7, r8 = blockIdx.x >> 3;
    const uint32_t item = r8 % n_items, tg = (r8 / n_items) * 8 + xcd;
    if (tg >= a.tgroups) return;  // whole workgroup

    const uint32_t lane = threadIdx.x & 63;
    const uint32_t n = lane & 15, g = lane >> 4;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t ts = wave / KS, ks = wave % KS;
    const uint32_t tile = tg * kTpw + ts;
    const uint32_t first = item * kGRows, count = min(a.batch - first, kGRows);
    const uint32_t nblk = a.units * 2;  // <= kGChunkBlocks (host)

    // ---- Activation loads first. Pass p of wave w covers block
    // b = w + kWaves p of the item's 8 rows: lane l holds row j = l / 8,
    // columns 4 (l % 8) .. + 3 of the block, one 16-byte load (cols is a
    // multiple of 32, so a quad is wholly inside or outside the row; outside
    // reads zeros; rows past the item read zeros).
    const uint32_t j = lane >> 3, jq = lane & 7;
    const BufRsrc x_r = make_rsrc(a.x, a.x_bytes);
    const uint32_t x_row = (first + j) * a.x_stride * 4 + 16 * jq;  // < 2^31 where used (host)
    float xv[kPasses][4];
#pragma unroll
    for (uint32_t p = 0; p < kPasses; ++p) {
        const uint32_t b = wave + kWaves * p;
        const bool ok = j < count && b * 32 + 4 * jq < a.cols;
        const uint4 v = buf_load_b128(x_r, ok ? x_row + b * 128 : kBufOob, 0);
        xv[p][0] = __uint_as_float(v.x);
        xv[p][1] = __uint_as_float(v.y);
        xv[p][2] = __uint_as_float(v.z);
        xv[p][3] = __uint_as_float(v.w);
    }
    __builtin_amdgcn_s_barrier();  // every wave's activation loads ahead of the weights

    // ---- This wave's weight steps, all in flight at once.
    const uint32_t upk = a.units / KS, steps = upk / UPS;  // steps <= 2 (host)
    const uint32_t u0 = ks * upk;
    const BufRsrc rec_r = make_rsrc(a.recs + a.mat * a.rec_stride, (uint32_t)(a.rec_stride * 16));
    const BufRsrc d_r = make_rsrc(a.dvals + a.mat * a.d_stride, (uint32_t)(a.d_stride * 2));
    const uint32_t rec_voff = lane * 16, d_voff = n * a.d_row * 2;
    const bool tile_ok = tile < a.tiles;
    uint4 rr[2][kMaxUnitsPerStep];
    uint32_t dd[2][kMaxUnitsPerStep];
#pragma unroll
    for (uint32_t s = 0; s < 2; ++s) {
        const uint32_t u = u0 + s * UPS;
        const bool ok = tile_ok && s < steps;
        load_step<kFmtQ8, UPS>(rec_r, rec_voff, ok ? (tile * a.units + u) * 1024 : kBufOob, d_r, d_voff,
                               ok ? (tile * 16 * a.d_row + 2 * u) * 2 : kBufOob, rr[s], dd[s]);
    }

    // ---- Quantise the item's rows into the LDS A layout: A row 2j / 2j + 1
    // = row j's hi / lo digits; lane (n, g) of block pair bp holds columns
    // 8g .. 8g + 7 of blocks 2 bp (bytes 0..7) and 2 bp + 1 (bytes 8..15).
    uint8_t* const a_lane = aq + ((jq >> 1) * 16 + 2 * j) * 16 + (jq & 1) * 4;
#pragma unroll
    for (uint32_t p = 0; p < kPasses; ++p) {
        const uint32_t b = wave + kWaves * p;
        if (b < nblk) {  // whole wave (blocks past the padded row are never read)
            uint32_t h4, l4;
            const float sc = quantize_quad(xv[p], h4, l4);
            uint8_t* const dst = a_lane + (b >> 1) * 1024 + (b & 1) * 8;
            *reinterpret_cast<uint32_t*>(dst) = h4;
            *reinterpret_cast<uint32_t*>(dst + 16) = l4;
            if (jq == 0) xs_lds[j * kGChunkBlocks + b] = sc;
        }
    }
    lds_barrier();

    float acc0 = 0.0f, acc1 = 0.0f;
    const float* xs0 = xs_lds + (2 * g) * kGChunkBlocks;
    const float* xs1 = xs0 + kGChunkBlocks;
#pragma unroll
    for (uint32_t s = 0; s < 2; ++s)
        if (s < steps) step_group_q8<UPS>(rr[s], dd[s], u0 + s * UPS, aq, xs0, xs1, lane, acc0, acc1);

    if (KS > 1) {
        if (ks > 0) {
            float* rp = red + ((ts * (KS - 1) + (ks - 1)) * 2) * 64;
            rp[lane] = acc0;
            rp[64 + lane] = acc1;
        }
        lds_barrier();
        if (ks > 0) return;
#pragma unroll
        for (uint32_t k = 1; k < KS; ++k) {
            const float* rp = red + ((ts * (KS - 1) + (k - 1)) * 2) * 64;
            acc0 += rp[lane];
            acc1 += rp[64 + lane];
        }
    }
    const uint32_t row = tile * 16 + n;
    if (tile_ok && row < a.rows) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t jr = 2 * g + h;
            if (jr < count) a.y[(uint64_t)(first + jr) * a.y_slot + (uint64_t)row * a.y_row] = h ? acc1 : acc0;
        }
    }
}

template <int FMT, int WG>
const void* group_kernel_for(int ups) {
    switch (ups) {
        case 1: return reinterpret_cast<const void*>(&group_kernel<FMT, 1, WG>);
        case 2: return reinterpret_cast<const void*>(&group_kernel<FMT, 2, WG>);
        case 3: return reinterpret_cast<const void*>(&group_kernel<FMT, 3, WG>);
        default: return reinterpret_cast<const void*>(&group_kernel<FMT, 4, WG>);
    }
}

int env_int(const char* name, int dflt) {
    const char* e = getenv(name);
    return e ? atoi(e) : dflt;
}

// Units per step: the largest of 4, 3, 2, 1 (with `most` below 4: of most
// and below) dividing both the tile's units and a chunk's (Q8_0 tiles hold a
// multiple of 4 units). Override: MMHIP_GROUP_UPS (1..4).
int group_ups(uint32_t units, uint32_t fmt, int most) {
    const uint32_t per_chunk = kGChunkBlocks / (fmt == kFmtIq2 ? 8 : 2);
    const uint32_t cu = units < per_chunk ? units : per_chunk;
    static const int most_env = env_int("MMHIP_GROUP_UPS", 0);
    if (most_env >= 1 && most_env <= 4) most = most_env;
    for (int u = most < 1 || most > 4 ? 4 : most; u >= 1; --u)
        if (units % u == 0 && cu % u == 0) return u;
    return 1;
}

int resident(const void* fn, int wg) {
    static std::mutex mu;
    static std::map<const void*, int> cache;
    std::lock_guard<std::mutex> lock(mu);
    auto it = cache.find(fn);
    if (it != cache.end()) return it->second;
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, fn, wg, 0) != hipSuccess || nb <= 0) nb = 1;
    cache[fn] = nb;
    return nb;
}

hipError_t launch(GroupArgs a, uint32_t fmt, uint32_t items, int num_cu, hipStream_t s) {
    if (items == 0 || a.tiles == 0) return hipSuccess;
    // Workgroup size and step, measured on MI355X at batch 64: IQ2_XXS
    // grouped experts run ~10% faster with 512 threads and one-unit steps
    // (four waves per SIMD; two-unit steps need 128 registers and spill)
    // than with 256 threads and four-unit steps, and 4% faster again with
    // one 1024-thread workgroup per CU than with two of 512. Of two
    // workgroups sharing a CU the older one was served first and ended ~10
    // us before the other (s_memrealtime per workgroup), which then ran
    // alone on the CU at half the waves. Each size needs its threads' worth
    // of tiles per CU (16 or 8 waves' worth); smaller calls (an MLA
    // projection at 64 tokens) would leave CUs idle and keep 256 threads.
    // Q8_0 is fastest with 256 / 4.
    // Override: MMHIP_GROUP_WG (256 | 512 | 1024, the last IQ2_XXS only).
    static const int wg_env = env_int("MMHIP_GROUP_WG", 0);
    const uint64_t cus = (uint64_t)(num_cu > 0 ? num_cu : 256);
    const uint64_t tiles_all = (uint64_t)items * a.tiles;
    const bool wg_ok = wg_env == 256 || wg_env == 512 || (wg_env == 1024 && fmt == kFmtIq2);
    const int wg = wg_ok                                         ? wg_env
                   : fmt == kFmtIq2 && tiles_all >= cus * 16 ? 1024
                   : fmt == kFmtIq2 && tiles_all >= cus * 8  ? 512
                                                                 : 256;
    const int ups = group_ups(a.units, fmt, wg >= 512 ? 1 : 4);
    const void* fn = fmt == kFmtIq2
                         ? (wg == 1024 ? group_kernel_for<kFmtIq2, 1024>(ups)
                            : wg == 512 ? group_kernel_for<kFmtIq2, 512>(ups)
                                        : group_kernel_for<kFmtIq2, 256>(ups))
                         : (wg == 512 ? group_kernel_for<kFmtQ8, 512>(ups) : group_kernel_for<kFmtQ8, 256>(ups));
    // Every resident workgroup slot of the device, or fewer when the largest
    // possible call has under one tile per wave for each of them; each
    // workgroup takes 1 / grid of the items' tiles (the actual item count
    // of a grouped call is only known on the device).
    const uint32_t waves = wg / 64;
    // An item switch costs a 1024-thread workgroup ~5.5 steps per wave
    // (batch-64 MoE layer, both grouped launches); in tiles of a workgroup's
    // range that is 5.5 x waves / (steps per tile). Measured there: 1.34 ->
    // 1.27 us per token. Dense calls with 256 threads (the MLA projections at
    // 64 tokens) ran slower with such a gap (48.5 -> 58.0 us per layer) and
    // keep ranges of equal tiles. MMHIP_GROUP_SWITCH_TENTHS: the cost in
    // tenths of a step (0: equal tiles).
    static const int sw_env = env_int("MMHIP_GROUP_SWITCH_TENTHS", 55);
    const uint64_t steps_per_tile = a.units / (uint32_t)ups > 0 ? a.units / (uint32_t)ups : 1;
    a.gap = (sw_env > 0 && wg == 1024 && a.work)
                ? (uint32_t)(((uint64_t)sw_env * waves + 5 * steps_per_tile) / (10 * steps_per_tile))
                : 0u;
    const uint64_t slots = cus * resident(fn, wg);
    const uint64_t most = ((uint64_t)items * a.tiles + waves - 1) / waves;
    const dim3 grid((unsigned)(most < slots ? most : slots));
    void* args[] = {&a};
    return hipLaunchKernel(fn, grid, dim3(wg), args, 0, s);
}

GroupArgs base(const uint4* recs, const uint16_t* dvals, const TileGeom& g, const QuantAct& xq, float* y) {
    GroupArgs a{};
    a.recs = recs;
    a.dvals = dvals;
    a.rec_stride = g.rec_stride;
    a.d_stride = g.d_stride;
    a.d_row = (uint32_t)g.d_row;
    a.xh = xq.hi;
    a.xl = xq.lo;
    a.xs = xq.scale;
    a.xq_stride = xq.stride;
    a.xs_stride = xq.scale_stride;
    a.y = y;
    a.tiles = (uint32_t)g.tiles;
    a.units = (uint32_t)g.units;
    a.rows = (uint32_t)g.rows;
    return a;
}

}  // namespace

hipError_t launch_group_dense(const uint4* recs, const uint16_t* dvals, const TileGeom& g, uint64_t mat,
                              const QuantAct& xq, uint32_t batch, float* y, uint64_t y_ld, int out_layout,
                              int num_cu, hipStream_t s) {
    if (batch == 0) return hipSuccess;
    GroupArgs a = base(recs, dvals, g, xq, y);
    a.mat = mat;
    a.batch = batch;
    a.y_slot = out_layout == 0 ? y_ld : 1;
    a.y_row = out_layout == 0 ? 1 : y_ld;
    return launch(a, g.fmt, (batch + kGRows - 1) / kGRows, num_cu, s);
}

// K slices per tile for the fused Q8_0 matmul: slices of two four-unit steps
// where the units split that way, else of one step (16 / slices tiles per
// workgroup); 0 for K above one LDS chunk (2048 columns) or units not a
// multiple of four.
static uint32_t qmm_q8_slices(const TileGeom& g) {
    if (g.fmt != kFmtQ8 || g.units == 0 || g.units * 2 > kGChunkBlocks || g.units % 4) return 0;
    return (uint32_t)(g.units % 8 == 0 ? g.units / 8 : g.units / 4);  // 1..7 (units <= 32)
}

bool qmm_q8_fused_fits(const TileGeom& g) { return qmm_q8_slices(g) != 0; }

hipError_t launch_qmm_q8_fused(const uint4* recs, const uint16_t* dvals, const TileGeom& g, uint64_t mat,
                               const float* x, uint64_t x_stride, uint32_t cols, uint32_t batch, float* y,
                               uint64_t y_ld, int out_layout, hipStream_t s) {
    if (batch == 0) return hipSuccess;
    const uint32_t ks = qmm_q8_slices(g);
    // x is addressed with 32-bit byte offsets from one buffer resource.
    const uint64_t x_bytes = ((uint64_t)(batch - 1) * x_stride + cols) * 4;
    if (ks == 0 || cols > g.cols_pad || cols % 32 || x_stride < cols || g.tiles == 0 || x_bytes >= kBufOob)
        return hipErrorInvalidValue;
    QmmQ8Args a{};
    a.recs = recs;
    a.dvals = dvals;
    a.rec_stride = g.rec_stride;
    a.d_stride = g.d_stride;
    a.d_row = (uint32_t)g.d_row;
    a.x = x;
    a.x_stride = (uint32_t)x_stride;
    a.x_bytes = (uint32_t)x_bytes;
    a.cols = cols;
    a.y = y;
    a.y_slot = out_layout == 0 ? y_ld : 1;
    a.y_row = out_layout == 0 ? 1 : y_ld;
    a.mat = mat;
    a.batch = batch;
    a.tiles = (uint32_t)g.tiles;
    a.units = (uint32_t)g.units;
    a.rows = (uint32_t)g.rows;
    const uint32_t tpw = 16 / ks;
    a.tgroups = (a.tiles + tpw - 1) / tpw;
    const uint64_t items = (batch + kGRows - 1) / kGRows;
    const uint64_t groups8 = (a.tgroups + 7) / 8;
    const uint64_t blocks = groups8 * items * 8;
    if (blocks > 0x7FFFFFFFu) return hipErrorInvalidValue;
    const void* fns[8] = {nullptr,
                          reinterpret_cast<const void*>(&qmm_q8_fused_kernel<1>),
                          reinterpret_cast<const void*>(&qmm_q8_fused_kernel<2>),
                          reinterpret_cast<const void*>(&qmm_q8_fused_kernel<3>),
                          reinterpret_cast<const void*>(&qmm_q8_fused_kernel<4>),
                          reinterpret_cast<const void*>(&qmm_q8_fused_kernel<5>),
                          reinterpret_cast<const void*>(&qmm_q8_fused_kernel<6>),
                          reinterpret_cast<const void*>(&qmm_q8_fused_kernel<7>)};
    void* args[] = {&a};
    return hipLaunchKernel(fns[ks], dim3((unsigned)blocks), dim3(tpw * ks * 64), args, 0, s);
}

hipError_t launch_group_experts(const uint4* recs, const uint16_t* dvals, const TileGeom& g, const QuantAct& xq,
                                const uint32_t* a_row, const QmmWork* work, const uint32_t* n_work, uint32_t max_work,
                                float* y, uint64_t y_ld, int num_cu, hipStream_t s) {
    GroupArgs a = base(recs, dvals, g, xq, y);
    a.work = work;
    a.n_work = n_work;
    a.a_row = a_row;
    a.y_slot = y_ld;
    a.y_row = 1;
    return launch(a, g.fmt, max_work, num_cu, s);
}

}  // namespace mmhip
