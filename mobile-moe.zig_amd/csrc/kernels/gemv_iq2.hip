// IQ2_XXS decode GEMV on gfx950 (matVecMulUnified's non-Q8_0 branch,
// inference.zig:1222-1226, and the expert products of expertFFN,
// inference.zig:1171-1185, without the f32 dequantization round trip).
//
// A workgroup owns one problem (matrix + activation vector) and up to
// IqShape::kMaxTiles 16-row tiles (kMaxItems record units per activation
// chunk): two 768-thread workgroups per CU by default, or one of 1024 threads
// (IqShape). A launch may hold several segments (weights of different
// shapes), each one slice (blockIdx.z) of the grid. The activation is quantised into
// LDS per K-chunk of up to 8 record units (2048 columns) as two int8 digit
// planes per 32-column block (x ~ s (256 hi + lo)).
//
// Work items are (unit, tile) pairs in unit-major order, split into equal
// contiguous runs, one per wave, so a wave keeps one unit's activation
// operands in registers while it walks tiles. In the 1024-thread shape the
// table reads of item i + 1 are issued before item i's arithmetic, so their
// latency overlaps it (two sets of table words in registers); the 768-thread
// shape hides it with its 24 waves per CU instead. The A operands are sparse: for
// the 16x16x64 MFMA of blocks 2j, 2j + 1 (lane group g's K range carries
// the record of sub-block 2j, then that of 2j + 1, both at columns
// 8g..8g+7) only the lanes whose A row m = 4i + e belongs to one of those
// blocks hold digits in that block's half (e = 0/1: hi/lo digits of block i,
// e = 2/3: of block i + 4), all others hold zero. The four MFMAs of a unit
// accumulate into one result, whose D rows 4g..4g+3 in lane (g, n) are then
// the hi/lo dot products of blocks g and g + 4 of row n: no cross-lane
// gather, two digit combines per item, and lane (g, n) scales exactly the two
// sub-blocks whose ls bits its own record dwords carry.
//
// B operands come from the 32 KiB LDS table keyed by b012 | P | idx (record
// layout in device_common.hpp); the hi3 signs of the high dword come from an
// 8-entry mask table and are applied with one xor-add.
//
// Each item leaves its 64 lane partial sums in LDS (768 threads: the four
// lane groups of each row summed in registers first, in the same order);
// after a chunk, every output row adds its (unit, lane group) partials in a
// fixed order, so the result does not depend on timing or on the shape.
#include "device_common.hpp"
#include "kernels.hpp"
#include "route_ops.hpp"
#include "iq2_ops.hpp"

namespace mmhip {

namespace {

constexpr uint32_t kQChunkUnits = 8;                 // record units per activation chunk
constexpr uint32_t kQChunkBlocks = kQChunkUnits * 8;  // 32-column blocks per chunk

// Workgroup shapes. 1024 threads: one workgroup per CU (16 waves), each
// item's 64 lane partials kept in LDS. 768 threads: two workgroups per CU
// (24 waves), which the CU holds only at <= 80 VGPRs and <= 52 KB of LDS per
// workgroup, so an item's four lane groups are summed in registers (16 row
// values per item in LDS) and the next item's table reads are not issued
// ahead (one register set of table words).
template <int WG>
struct IqShape {
    static constexpr bool kPair = WG == 768;
    static constexpr uint32_t kWaves = WG / 64;
    static constexpr uint32_t kMaxTiles = kPair ? 32 : 64;    // row tiles per workgroup
    static constexpr uint32_t kMaxItems = kPair ? 192 : 384;  // (unit, tile) items per workgroup and chunk
    static constexpr uint32_t kPartPerItem = kPair ? 16 : 64;
};


// Activation columns [c0, c0 + 32 nblk) of the problem's vector (times
// silu(x) * u when silu_mul) into the digit planes; WG / 8 blocks per pass.
template <int WG>
__device__ __forceinline__ void quantize_planes(BufRsrc xr, BufRsrc ur, bool silu_mul, uint32_t nblk, uint8_t* aq,
                                                float* xs) {
    for (uint32_t b0 = 0; b0 < nblk; b0 += WG / 8) {
        float v[4], u[4];
        x_pass_load(xr, b0, v);
        x_pass_load(ur, b0, u);
        if (silu_mul) silu_mul4(v, u);
        x_store_planes(v, nblk, b0, aq, xs);
    }
}

// Problem p of the launch: matrix, activation row and output row; false when
// the problem does not run in this call.
template <bool ROUTE, class A>
__device__ __forceinline__ bool select_problem(const A& a, uint32_t p, uint64_t& mat, uint64_t& x_row,
                                               uint64_t& y_row) {
    mat = a.first_mat + p;
    x_row = p;
    y_row = p;
    if constexpr (ROUTE) {
        // Routes the token (run by one wave); the problem follows.
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
            return true;
        }
        if (a.route.shared && a.route.shared_merged && p < 2 * n_act + 2) {
            mat = 2 * E + (p - 2 * n_act);
            y_row = 8 + (p - 2 * n_act);
            return true;
        }
        return false;
    } else {
        return read_problem(a.probs, a.n_active, p, mat, x_row, y_row);
    }
}

// Position of an item: unit ul within the chunk, tile t within the
// workgroup's range (unit-major order).
struct ItemPos {
    uint32_t ul, t;
};


template <int DEPTH, bool ROUTE, int NSEG, int WG, class A>
__device__ __forceinline__ void gemv_iq2_body(const A& a, const GemvArgs& lt) {
    using Shape = IqShape<WG>;
    constexpr bool kPair = Shape::kPair;
    constexpr uint32_t kWaves = Shape::kWaves;
    constexpr int kRing = DEPTH + 1;
    static_assert(kPair || kRing % 2 == 0, "two table-word sets alternate over the ring");
    // One LDS block with the table first: its byte offsets (below 32 KiB)
    // fold into the ds_read offset fields.
    struct Lds {
        uint32_t tab[kIq2TableWords];
        uint32_t mtab[8];  // hi3 sign masks
        // Per item: row n's lane groups g at 4 n + g, or (kPair) row n's sum
        // over its lane groups at n.
        alignas(16) float part[Shape::kMaxItems * Shape::kPartPerItem];
        uint8_t aq[kQChunkBlocks * 64];
        float xs[kQChunkBlocks];
        uint32_t sel[2];  // ROUTE: the routed problem's matrix (~0u: none) and output row
    };
    static_assert(!kPair || sizeof(Lds) <= 52 * 1024, "two workgroups per CU need <= 52 KB of LDS each");
    // Thread i owns output row i of the workgroup's range: its sum over the
    // activation chunks stays in a register.
    static_assert(Shape::kMaxTiles * 16 <= WG, "one output row per thread");
    __shared__ __align__(16) Lds lds;
    uint32_t* const tab = lds.tab;
    const uint32_t* const mtab = lds.mtab;
    float* const part = lds.part;
    uint8_t* const aq = lds.aq;
    float* const xs = lds.xs;

    // This workgroup's problem within its segment (row y); a: the segment.
    const uint32_t py = blockIdx.y;
    const uint32_t t_begin = blockIdx.x * a.tiles_per_wg;
    // The grid is sized for the widest and longest segment.
    if (t_begin >= a.tiles || py >= a.n_probs) return;  // whole workgroup

    const uint32_t lane = threadIdx.x & 63;
    const uint32_t n = lane & 15, g = lane >> 4;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // The problem: known up front, except in the decode gate/up variant,
    // where wave 0 routes the token after every wave's table and activation
    // loads (row 0) are issued, so the routing overlaps their latency (one
    // wave: sixteen waves routing the same token cost ~2 us of issue time).
    uint64_t mat = 0, x_row = 0, y_row = 0;
    if constexpr (!ROUTE) {
        if (!select_problem<false>(a, py, mat, x_row, y_row)) return;  // whole workgroup
    }
    const float* x = a.x + x_row * a.x_stride;
    float* y_base = nullptr;
    const bool silu_mul = a.silu_mul != 0;
    const uint32_t n_tiles = min(a.tiles - t_begin, a.tiles_per_wg);
    BufRsrc rec_r, d_r;
    const uint32_t rec_voff = lane * 16;
    const uint32_t d_voff = n * a.d_row * 2;
    const uint32_t rec_tile = keep_sgpr(a.units * 1024u), d_tile = keep_sgpr(a.d_row * 32u);
    // This lane's word in an item's 64 partials: row-major (4 n + g), so the
    // row sums read each row's four lane groups as one 16-byte word.
    const uint32_t part_slot = (n << 2) | g;
    // Sparse A row of this lane: block s_star of the unit, digit d_star.
    const uint32_t s_star = (n >> 2) + 4 * ((n >> 1) & 1u), d_star = n & 1u;

    // Per-chunk state (set by start_chunk): items (unit ul, tile t), tp_n
    // tiles per unit, this wave's items [p0, p1).
    uint32_t u0 = 0, uc = 1, tp_n = 1, p0 = 0, p1 = 0;
    auto start_chunk = [&](uint32_t chunk_u0, uint32_t units_in_chunk) {
        u0 = chunk_u0;
        uc = units_in_chunk;
        tp_n = n_tiles;
        const uint32_t N = uc * tp_n;
        p0 = wave * N / kWaves;
        p1 = (wave + 1) * N / kWaves;
    };
    auto advance = [&](ItemPos q) { return (q.t + 1 == tp_n) ? ItemPos{q.ul + 1, 0} : ItemPos{q.ul, q.t + 1}; };
    // Loads item q (ItemPos.t = tile within the range).
    auto load = [&](bool valid, ItemPos q, uint4& r, uint16_t& dbits) {
        uint32_t rs = kBufOob, ds = kBufOob;
        if (valid) {
            const uint32_t tile = t_begin + q.t, u = u0 + q.ul;
            rs = tile * rec_tile + u * 1024;
            ds = tile * d_tile + u * 2;
        }
        r = buf_load_b128<kCacheStream>(rec_r, rec_voff, rs);
        dbits = buf_load_b16(d_r, d_voff, ds);  // cached: the tile's other units reuse the line
    };

    uint4 rb[kRing];
    uint16_t db[kRing];
    ItemPos cur{0, 0}, nxt{0, 0};
    auto issue_first = [&]() {
        cur = ItemPos{p0 / tp_n, p0 % tp_n};
        nxt = cur;
#pragma unroll
        for (int q = 0; q < DEPTH; ++q) {
            load(p0 + q < p1, nxt, rb[q], db[q]);
            nxt = advance(nxt);
        }
    };

    {
        // Prologue: tables and the first activation chunk load, every wave's
        // loads issued (barrier) before any weight load, then the first
        // weight items go out while LDS is filled.
        const uint32_t uc0 = min(a.units, kQChunkUnits);
        const uint32_t nb = uc0 * 8;
        const uint32_t xb = min(a.cols, nb * 32) * 4;
        const BufRsrc x_r = make_rsrc(x, xb);
        const BufRsrc u_r = make_rsrc(x + a.x2_off, silu_mul ? xb : 0);  // zero-size: loads read 0
        const BufRsrc t_r = make_rsrc(&c_iq2_tables, sizeof(Iq2Tables));
        constexpr uint32_t kTabVecs = kIq2TableWords / 4, kTabPer = (kTabVecs + WG - 1) / WG;
        uint4 tv[kTabPer];
#pragma unroll
        for (uint32_t i = 0; i < kTabPer; ++i) tv[i] = buf_load_b128(t_r, (threadIdx.x + WG * i) * 16, 0);
        float xv[4], uv[4];
        x_pass_load(x_r, 0, xv);
        x_pass_load(u_r, 0, uv);
        if constexpr (ROUTE) {
            // Wave 0 routes the token and hands the problem to the others
            // through LDS; the barrier also orders every wave's loads above
            // before its weight loads.
            if (wave == 0) {
                const bool run = select_problem<true>(a, py, mat, x_row, y_row);
                if (lane == 0) {
                    lds.sel[0] = run ? (uint32_t)mat : ~0u;
                    lds.sel[1] = (uint32_t)y_row;
                }
            }
            lds_barrier();
            const uint32_t sel = lds.sel[0];
            if (sel == ~0u) return;  // whole workgroup; x_row stays 0
            mat = sel;
            y_row = lds.sel[1];
        }
        y_base = lt.y + y_row * lt.y_stride;
        rec_r = make_rsrc(a.recs + mat * a.rec_stride, (uint32_t)(a.rec_stride * 16));
        d_r = make_rsrc(a.dvals + mat * a.d_stride, (uint32_t)(a.d_stride * 2));
        start_chunk(0, uc0);
        if constexpr (!ROUTE) __builtin_amdgcn_s_barrier();
        issue_first();
#pragma unroll
        for (uint32_t i = 0; i < kTabPer; ++i)
            if (kTabVecs % WG == 0 || threadIdx.x + WG * i < kTabVecs)
                reinterpret_cast<uint4*>(tab)[threadIdx.x + WG * i] = tv[i];
        if (threadIdx.x < 8) {
            // Columns 4..6 take hi3's bits, column 7 its parity (the ksigns
            // parity bit; column 7's P sign is already in the table word).
            lds.mtab[threadIdx.x] = iq2_hi3_mask(threadIdx.x);
        }
        if (silu_mul) silu_mul4(xv, uv);
        static_assert(WG / 8 >= kQChunkBlocks, "one pass quantises the first chunk");
        x_store_planes(xv, nb, 0, aq, xs);
    }

    float row_acc = 0.0f;  // this thread's output row, summed over the chunks
    for (uint32_t kc = 0;;) {
        lds_barrier();  // tables, digit planes and scales visible
        v4i av[4];
        float xa = 0.0f, xb = 0.0f, ha = 0.0f, hb = 0.0f;
        uint32_t a_ul = 0xFFFFFFFFu;
        // This unit's sparse A operands and block scales.
        auto set_unit = [&](uint32_t ul) {
            a_ul = ul;
            const uint8_t* ap = aq + ((a_ul * 8 + s_star) * 2 + d_star) * 32 + 8 * g;
            const uint2 xw = *reinterpret_cast<const uint2*>(ap);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const bool lo = s_star == 2u * j, hi = s_star == 2u * j + 1;
                av[j] = v4i{(int)(lo ? xw.x : 0u), (int)(lo ? xw.y : 0u), (int)(hi ? xw.x : 0u), (int)(hi ? xw.y : 0u)};
            }
            xa = xs[a_ul * 8 + g] * 0.25f;
            xb = xs[a_ul * 8 + g + 4] * 0.25f;
            ha = xa * 0.5f;
            hb = xb * 0.5f;
        };
        // Lane (g, n)'s partial of row n for the item in ring slot q, whose
        // table words (signs applied) are b.
        auto item_value = [&](const RawB& b, int q) {
            v4i acc = {0, 0, 0, 0};
#pragma unroll
            for (int j = 0; j < 4; ++j) acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[j], b.e[j], acc, 0, 0, 0);
            // Blocks g and g + 4 of row n: d * (0.5 + ls) / 4 * s_x * digits.
            const uint4& r = rb[q];
            const float df = f16_scale(db[q]);
            const float sa = fmaf((float)iq2_ls_a(r), xa, ha);
            const float sb = fmaf((float)iq2_ls_b(r), xb, hb);
            float v = (float)digits_combine(acc[0], acc[1]) * sa;
            v = fmaf((float)digits_combine(acc[2], acc[3]), sb, v);
            return v * df;
        };
        // Issue priority by items left, set once per kRing items: the
        // hardware otherwise favours a SIMD's oldest wave, whose items then
        // finish far ahead of the youngest's, and the workgroup waits for the
        // last wave with the CU part idle.
        auto set_priority = [&](uint32_t rem) {
            if (rem > 8) __builtin_amdgcn_s_setprio(3);
            else if (rem > 4) __builtin_amdgcn_s_setprio(2);
            else if (rem > 2) __builtin_amdgcn_s_setprio(1);
            else __builtin_amdgcn_s_setprio(0);
        };
        if constexpr (kPair) {
            // Single items, table reads after the item's record arrives (one
            // register set); an item's lane groups summed in registers.
            for (uint32_t i = p0; i < p1; i += kRing) {
                set_priority(p1 - i);
#pragma unroll
                for (int q = 0; q < kRing; ++q) {
                    if (i + q < p1) {
                        load(i + q + DEPTH < p1, nxt, rb[(q + DEPTH) % kRing], db[(q + DEPTH) % kRing]);
                        nxt = advance(nxt);
                        RawB raw;
                        fetch_b(rb[q], tab, mtab, raw);
                        if (cur.ul != a_ul) set_unit(cur.ul);
                        finish_b(raw);
                        const float rv = item_rows(item_value(raw, q));
                        if (lane < 16) part[(cur.ul * n_tiles + cur.t) * 16 + n] = rv;
                        cur = advance(cur);
                    }
                }
            }
        } else {
            // Single items; the table reads of item i + 1 are issued before
            // item i's arithmetic (two register sets, kRing even keeps the
            // set of an item fixed at compile time).
            RawB raw[2];
            if (p0 < p1) fetch_b(rb[0], tab, mtab, raw[0]);
            for (uint32_t i = p0; i < p1; i += kRing) {
                set_priority(p1 - i);
#pragma unroll
                for (int q = 0; q < kRing; ++q) {
                    if (i + q < p1) {
                        load(i + q + DEPTH < p1, nxt, rb[(q + DEPTH) % kRing], db[(q + DEPTH) % kRing]);
                        nxt = advance(nxt);
                        if (i + q + 1 < p1) fetch_b(rb[(q + 1) % kRing], tab, mtab, raw[(q + 1) & 1]);
                        if (cur.ul != a_ul) set_unit(cur.ul);
                        finish_b(raw[q & 1]);
                        part[(cur.ul * n_tiles + cur.t) * 64 + part_slot] = item_value(raw[q & 1], q);
                        cur = advance(cur);
                    }
                }
            }
        }
        lds_barrier();  // every item's partials written
        // Row sums: units in order, lane groups in order (one 16-byte read
        // per unit, or the unit's row value already summed over its lane
        // groups in that order; a wave's lanes read consecutive words, no
        // bank conflicts).
        if (threadIdx.x < n_tiles * 16) {
            const uint32_t t = threadIdx.x >> 4, rr = threadIdx.x & 15;
            float sum = 0.0f;
            for (uint32_t ul = 0; ul < uc; ++ul) {
                if constexpr (kPair) {
                    sum += part[(ul * n_tiles + t) * 16 + rr];
                } else {
                    const float4 q = *reinterpret_cast<const float4*>(part + (ul * n_tiles + t) * 64 + rr * 4);
                    sum += ((q.x + q.y) + q.z) + q.w;
                }
            }
            row_acc += sum;
        }
        kc += uc;
        if (kc >= a.units) break;
        // Next K-chunk: re-quantise the activation (the planes and partials
        // are free once every wave passed the barrier below).
        lds_barrier();
        const uint32_t ucn = min(a.units - kc, kQChunkUnits);
        const uint32_t c0 = kc * 256;
        const uint32_t cb = (a.cols > c0 ? min(a.cols - c0, ucn * 256) : 0) * 4;
        quantize_planes<WG>(make_rsrc(x + c0, cb), make_rsrc(x + a.x2_off + c0, silu_mul ? cb : 0), silu_mul, ucn * 8,
                        aq, xs);
        start_chunk(kc, ucn);
        issue_first();
    }
    if (threadIdx.x < n_tiles * 16) {
        const uint32_t row = (t_begin + (threadIdx.x >> 4)) * 16 + (threadIdx.x & 15);
        if (row < lt.rows) y_base[row] = row_acc;
    }
}

template <int DEPTH, bool ROUTE, int NSEG, int WG = 1024>
__global__ __launch_bounds__(WG, IqShape<WG>::kPair ? 6 : 1) void gemv_iq2_kernel(GemvSet<NSEG> set) {
    // This workgroup's segment (grid slice z).
    const GemvArgs& a = set.seg[NSEG > 1 ? blockIdx.z : 0];
    pin_gemv_args(a);
    gemv_iq2_body<DEPTH, ROUTE, NSEG, WG>(a, a);
}

// One segment without a problem list or silu_mul (GemvOneArgs): the leading
// scalar arguments (14 dwords: tiles per workgroup and problems share one)
// are preloaded into SGPRs (GemvOneArgs, kernels.hpp).
template <int DEPTH, int WG>
__global__ __launch_bounds__(WG, IqShape<WG>::kPair ? 6 : 1) void gemv_iq2_one_kernel(
    const uint4* recs, const uint16_t* dvals, const float* x, uint32_t rec_stride, uint32_t d_stride, uint32_t x_stride,
    uint32_t cols, uint32_t units, uint32_t tpw_probs, uint32_t tiles, uint32_t d_row, GemvSet<1> set) {
    const GemvOneArgs a{recs,  dvals, x,     rec_stride,      d_stride,         x_stride, cols,
                        units, tpw_probs & 0xFFFFu, tiles, tpw_probs >> 16, d_row};
    gemv_iq2_body<DEPTH, false, 1, WG>(a, set.seg[0]);
}

static int env_int(const char* name, int dflt) {
    const char* e = getenv(name);
    return e ? atoi(e) : dflt;
}

// Largest tiles per workgroup for a segment: the LDS holds kMaxTiles row
// sums and kMaxItems (unit, tile) partials per activation chunk.
template <int WG>
static uint32_t max_tiles_per_wg(const GemvArgs& a) {
    const uint32_t uc = a.units < kQChunkUnits ? a.units : kQChunkUnits;
    uint32_t m = IqShape<WG>::kMaxItems / uc;
    if (m > IqShape<WG>::kMaxTiles) m = IqShape<WG>::kMaxTiles;
    return a.tiles < m ? a.tiles : m;
}

// Decode down projection and combine of one token (IQ2_XXS experts): the
// down GEMVs of every computed expert (up to kMaxK routed + the merged
// shared expert) and moeFFN's final sum (inference.zig:960-1010) in one
// launch. Workgroup t owns row tile t of every problem, so the weighted sum
// over the experts needs no other workgroup: all problems' weight loads and
// activation loads are issued up front, the activations silu(g) * u are
// quantised into LDS side by side (unit u' = p * units + u), each wave takes
// items (p, u) with the decode GEMV's arithmetic, and the tile's 16 rows are
// then summed per problem (units in order, lane groups in order, as the
// decode GEMV does) and combined in route order as combine_kernel does.
constexpr int kDcWg = 1024;
constexpr uint32_t kDcWaves = kDcWg / 64;
constexpr uint32_t kDcMaxProbs = kMaxK + 1;
constexpr uint32_t kDcMaxUnits = 8;  // inner width <= 2048
constexpr uint32_t kDcMaxItems = kDcMaxProbs * kDcMaxUnits;
constexpr uint32_t kDcItemsPerWave = (kDcMaxItems + kDcWaves - 1) / kDcWaves;


__global__ __launch_bounds__(kDcWg, 1) void down_combine_iq2_kernel(DownCombineArgs a) {
    struct Lds {
        uint32_t tab[kIq2TableWords];
        uint32_t mtab[8];
        uint8_t aq[kDcMaxItems * 8 * 64];
        float xs[kDcMaxItems * 8];
        alignas(16) float part[kDcMaxItems * 64];  // per item: row n's lane groups g at 4 n + g
        float ysum[kDcMaxProbs * 16];
        float cw[kMaxK];        // route weights of the computed entries
        int32_t cs[kMaxK + 1];  // their slots, then the shared slot (-1: none)
    };
    __shared__ __align__(16) Lds lds;
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t n = lane & 15, g = lane >> 4;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t tile = blockIdx.x;
    const uint32_t units = a.units, nblk = units * 8;
    // The count and the whole problem list in one round trip (the list
    // always has kDcMaxProbs entries; those past the count are ignored).
    uint4 prob[kDcMaxProbs];
#pragma unroll
    for (uint32_t p = 0; p < kDcMaxProbs; ++p) prob[p] = a.probs[p];
    const uint32_t n_act = min(*a.n_active, kDcMaxProbs);
    const uint32_t n_items = n_act * units;
    uint32_t slot[kDcMaxProbs];
#pragma unroll
    for (uint32_t p = 0; p < kDcMaxProbs; ++p) {
        if (p >= n_act) prob[p] = make_uint4(0, 0, 0xFFFFFFFFu, 0);
        slot[p] = prob[p].z;
    }

    // Small loads first: tables, every problem's activation pair.
    constexpr int kTabPer = kIq2TableWords / 4 / kDcWg;
    const BufRsrc t_r = make_rsrc(&c_iq2_tables, sizeof(Iq2Tables));
    uint4 tv[kTabPer];
#pragma unroll
    for (int i = 0; i < kTabPer; ++i) tv[i] = buf_load_b128(t_r, (threadIdx.x + kDcWg * i) * 16, 0);
    // The combine's inputs, read now so their latency overlaps the loads.
    const uint32_t row = tile * 16 + (threadIdx.x & 15);
    const float bias_v = (a.bias && threadIdx.x < 16 && row < a.rows) ? a.bias[row] : 0.0f;
    const uint32_t deferred = a.deferred[0];
    float cw = 0.0f;
    int32_t cs = -1;
    if (threadIdx.x < kMaxK) {
        cs = a.assign_slot[threadIdx.x];
        cw = a.assign_w[threadIdx.x];
    } else if (threadIdx.x == kMaxK) {
        cs = a.shared_slot[0];
    }
    // The problems' blocks side by side: global block B = p * nblk + b, 8
    // lanes (4 columns each) per block, kDcWg / 8 blocks per pass.
    constexpr uint32_t kPassBlocks = kDcWg / 8;
    constexpr uint32_t kPasses = (kDcMaxItems * 8 + kPassBlocks - 1) / kPassBlocks;
    const uint32_t xbytes = (uint32_t)((kDcMaxProbs * a.x_stride) * 4);
    const BufRsrc xr = make_rsrc(a.x, xbytes);
    float xv[kPasses][4], uv[kPasses][4];
#pragma unroll
    for (uint32_t q = 0; q < kPasses; ++q) {
        const uint32_t B = q * kPassBlocks + (threadIdx.x >> 3);
        const uint32_t p = B / nblk, c = (B - p * nblk) * 32 + 4 * (threadIdx.x & 7);
        uint32_t xrow = 0;
#pragma unroll
        for (uint32_t r = 0; r < kDcMaxProbs; ++r)
            if (r == p) xrow = prob[r].y;
        const bool ok = p < n_act && c < a.cols;
        const uint32_t o0 = ok ? (uint32_t)((xrow * a.x_stride + c) * 4) : kBufOob;
        const uint32_t o1 = ok ? (uint32_t)((xrow * a.x_stride + a.x2_off + c) * 4) : kBufOob;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            xv[q][e] = __uint_as_float(buf_load_b32(xr, o0 + 4 * e, 0));
            uv[q][e] = __uint_as_float(buf_load_b32(xr, o1 + 4 * e, 0));
        }
    }
    // Every wave's small loads are issued before any weight load: a CU
    // returns loads in issue order.
    __builtin_amdgcn_s_barrier();
    // Weight items of this wave: item i = p * units + u, i = wave + kDcWaves j.
    uint4 rb[kDcItemsPerWave];
    uint16_t db[kDcItemsPerWave];
    const uint32_t rec_voff = lane * 16, d_voff = n * a.d_row * 2;
#pragma unroll
    for (uint32_t j = 0; j < kDcItemsPerWave; ++j) {
        const uint32_t i = wave + kDcWaves * j;
        const bool ok = i < n_items;
        const uint32_t p = ok ? i / units : 0, u = i - p * units;
        uint64_t mat = 0;
#pragma unroll
        for (uint32_t q = 0; q < kDcMaxProbs; ++q)
            if (ok && q == p) mat = prob[q].x;
        const BufRsrc rr = make_rsrc(a.recs + mat * a.rec_stride, (uint32_t)(a.rec_stride * 16));
        const BufRsrc dr = make_rsrc(a.dvals + mat * a.d_stride, (uint32_t)(a.d_stride * 2));
        rb[j] = buf_load_b128<kCacheStream>(rr, rec_voff, ok ? (tile * units + u) * 1024 : kBufOob);
        db[j] = buf_load_b16(dr, d_voff, ok ? (tile * 16 * a.d_row + u) * 2 : kBufOob);
    }
#pragma unroll
    for (int i = 0; i < kTabPer; ++i) reinterpret_cast<uint4*>(lds.tab)[threadIdx.x + kDcWg * i] = tv[i];
    if (threadIdx.x < 8) lds.mtab[threadIdx.x] = iq2_hi3_mask(threadIdx.x);
    if (threadIdx.x <= kMaxK) {
        lds.cs[threadIdx.x] = cs;
        if (threadIdx.x < kMaxK) lds.cw[threadIdx.x] = cw;
    }
#pragma unroll
    for (uint32_t q = 0; q < kPasses; ++q) {
        if (q * kPassBlocks >= n_items * 8) break;  // uniform
#pragma unroll
        for (int e = 0; e < 4; ++e) xv[q][e] = silu_fast(xv[q][e]) * uv[q][e];
        // Every thread quantises (the block max uses DPP); blocks of
        // problems that run are stored.
        x_store_planes(xv[q], n_items * 8, q * kPassBlocks, lds.aq, lds.xs);
    }
    lds_barrier();

#pragma unroll
    for (uint32_t j = 0; j < kDcItemsPerWave; ++j) {
        const uint32_t i = wave + kDcWaves * j;
        if (i >= n_items) break;
        lds.part[i * 64 + ((n << 2) | g)] = iq2_item(rb[j], db[j], lds.aq + i * 8 * 64, lds.xs + i * 8, lds.tab, lds.mtab, n, g);
    }
    lds_barrier();
    if (threadIdx.x < 16 * kDcMaxProbs) {
        // Row r of problem p: the decode GEMV's row sum (units, then lane
        // groups, in order, added to a zero row).
        const uint32_t p = threadIdx.x >> 4, r = threadIdx.x & 15;
        if (p < n_act) {
            float sum = 0.0f;
            for (uint32_t u = 0; u < units; ++u) {
                const float4 q = *reinterpret_cast<const float4*>(lds.part + (p * units + u) * 64 + r * 4);
                sum += ((q.x + q.y) + q.z) + q.w;
            }
            lds.ysum[p * 16 + r] = 0.0f + sum;
        }
    }
    lds_barrier();
    if (threadIdx.x < 16 && row < a.rows) {
        // Slot s (route order, shared last) -> its problem's row value.
        auto slot_val = [&](int32_t s) {
            float v = 0.0f;
            for (uint32_t p = 0; p < n_act; ++p)
                if (slot[p] == (uint32_t)s) v = lds.ysum[p * 16 + threadIdx.x];
            return v;
        };
        float o = 0.0f;
#pragma unroll
        for (int i = 0; i < kMaxK; ++i) {
            const int32_t sl = lds.cs[i];
            if (sl >= 0) o = __fadd_rn(o, __fmul_rn(lds.cw[i], slot_val(sl)));
        }
        const int32_t sh = lds.cs[kMaxK];
        if (sh >= 0) o = __fadd_rn(o, slot_val(sh));
        if (a.bias && deferred) o = __fadd_rn(o, bias_v);
        a.out[row] = o;
    }
}

template <int N>
static hipError_t launch_set(const GemvArgs* segs, uint32_t n_segs, const void* fn, uint32_t grid_x, uint32_t wg,
                             hipStream_t s) {
    GemvSet<N> set{};
    uint32_t y = 0;
    for (uint32_t i = 0; i < (uint32_t)N; ++i) {
        set.seg[i] = segs[i < n_segs ? i : 0];
        if (i < n_segs && segs[i].n_probs > y) y = segs[i].n_probs;
    }
    void* args[] = {&set};
    return hipLaunchKernel(fn, dim3(grid_x, y, n_segs), dim3(wg), args, 0, s);
}

// Tiles per workgroup of every segment and the grid's x extent for W
// workgroups of shape WG, `slots` of which fit the GPU at once.
template <int WG>
static uint32_t plan_tiles(GemvArgs* segs, uint32_t n, uint64_t slots) {
    uint32_t grid_x = 1;
    if (n == 1) {
        // Tiles per workgroup. A grid of W workgroups runs in
        // ceil(W / slots) rounds; the choice minimises rounds x (tiles x
        // units x per-item time + per-workgroup fixed time), with the costs
        // measured on MI355X for one 1024-thread workgroup per CU (~65 ns per
        // 1 KiB item per CU, ~2 us of prologue and tail). E.g. 10 matrices
        // of 128 tiles take 6 tiles per workgroup (220 workgroups, one round)
        // rather than 5 (260, two rounds).
        GemvArgs& a = segs[0];
        const uint32_t max_tpw = max_tiles_per_wg<WG>(a);
        uint32_t tpw = max_tpw;
        double best = 0.0;
        for (uint32_t t = 1; t <= max_tpw; ++t) {
            const uint64_t wgs = (uint64_t)a.n_probs * ((a.tiles + t - 1) / t);
            const double cost = (double)((wgs + slots - 1) / slots) * ((double)t * a.units * 0.065 + 2.0);
            if (t == 1 || cost < best) {
                best = cost;
                tpw = t;
            }
        }
        a.tiles_per_wg = tpw;
        grid_x = (a.tiles + tpw - 1) / tpw;
    } else {
        // Several segments: every workgroup gets about the same number of
        // items (the total over the slots), so the whole launch is one round
        // when the segments allow it.
        uint64_t items = 0;
        for (uint32_t i = 0; i < n; ++i) items += (uint64_t)segs[i].n_probs * segs[i].tiles * segs[i].units;
        const uint64_t per_wg = (items + slots - 1) / slots;
        for (uint32_t i = 0; i < n; ++i) {
            GemvArgs& a = segs[i];
            uint64_t t = (per_wg + a.units - 1) / a.units;
            const uint32_t m = max_tiles_per_wg<WG>(a);
            if (t > m) t = m;
            if (t < 1) t = 1;
            a.tiles_per_wg = (uint32_t)t;
            const uint32_t gx = (a.tiles + a.tiles_per_wg - 1) / a.tiles_per_wg;
            if (gx > grid_x) grid_x = gx;
        }
    }
    return grid_x;
}

}  // namespace

hipError_t launch_gemv_iq2(const GemvArgs* segs_in, uint32_t n_segs, int num_cu, hipStream_t s) {
    if (n_segs == 0 || n_segs > kGemvMaxSegs) return hipErrorInvalidValue;
    GemvArgs segs[kGemvMaxSegs];
    uint32_t n = 0;
    for (uint32_t i = 0; i < n_segs; ++i)
        if (segs_in[i].n_probs && segs_in[i].tiles) segs[n++] = segs_in[i];
    if (n == 0) return hipSuccess;
    const bool route = segs[0].route_decode != 0;
    if (route && n != 1) return hipErrorInvalidValue;
    const uint64_t cus = (uint64_t)(num_cu > 0 ? num_cu : 256);
    // Two 768-thread workgroups per CU, or one of 1024 (MMHIP_IQ2_PAIR=0).
    // The 768-thread shape keeps one record load in flight per wave while
    // it computes another: with 24 waves per CU that is enough, and the
    // headline 64 + 64 matrix step ran ~0.5 us faster than with two (the
    // CU returns loads in issue order, so deeper prefetch only lengthens the
    // queue in front of the record a wave needs next).
    static const int pair_env = env_int("MMHIP_IQ2_PAIR", 1);
    if (pair_env != 0) {
        const uint32_t grid_x = plan_tiles<768>(segs, n, 2 * cus);
        const void* fn = route    ? reinterpret_cast<const void*>(&gemv_iq2_kernel<1, true, 1, 768>)
                         : n == 1 ? reinterpret_cast<const void*>(&gemv_iq2_kernel<1, false, 1, 768>)
                         : n == 2 ? reinterpret_cast<const void*>(&gemv_iq2_kernel<1, false, 2, 768>)
                                  : reinterpret_cast<const void*>(&gemv_iq2_kernel<1, false, 4, 768>);
        if (n == 1) {
            const GemvArgs& a = segs[0];
            if (!route && !a.probs && !a.n_active && !a.silu_mul && a.rec_stride < (1ull << 27) &&
                a.d_stride < (1ull << 30) && a.x_stride < (1ull << 32) && a.n_probs < 65536 && a.tiles_per_wg < 65536) {
                // Preloaded arguments (gemv_iq2_one_kernel).
                GemvSet<1> set{};
                set.seg[0] = a;
                const uint4* recs = a.recs + a.first_mat * a.rec_stride;
                const uint16_t* dvals = a.dvals + a.first_mat * a.d_stride;
                const float* x = a.x;
                uint32_t rs = (uint32_t)a.rec_stride, ds = (uint32_t)a.d_stride, xs = (uint32_t)a.x_stride;
                uint32_t cols = a.cols, units = a.units, tpw_np = a.tiles_per_wg | (a.n_probs << 16), tiles = a.tiles,
                         drow = a.d_row;
                void* args[] = {&recs, &dvals, &x, &rs, &ds, &xs, &cols, &units, &tpw_np, &tiles, &drow, &set};
                return hipLaunchKernel(reinterpret_cast<const void*>(&gemv_iq2_one_kernel<1, 768>),
                                       dim3(grid_x, a.n_probs, 1), dim3(768), args, 0, s);
            }
            return launch_set<1>(segs, 1, fn, grid_x, 768, s);
        }
        if (n == 2) return launch_set<2>(segs, 2, fn, grid_x, 768, s);
        return launch_set<4>(segs, n, fn, grid_x, 768, s);
    }
    const uint32_t grid_x = plan_tiles<1024>(segs, n, cus);
    // Items in flight per wave: 3 (the ring of record buffers is 4, even so
    // that an item's table-word set is fixed at compile time).
    const void* fn = route    ? reinterpret_cast<const void*>(&gemv_iq2_kernel<3, true, 1>)
                     : n == 1 ? reinterpret_cast<const void*>(&gemv_iq2_kernel<3, false, 1>)
                     : n == 2 ? reinterpret_cast<const void*>(&gemv_iq2_kernel<3, false, 2>)
                              : reinterpret_cast<const void*>(&gemv_iq2_kernel<3, false, 4>);
    if (n == 1) return launch_set<1>(segs, 1, fn, grid_x, 1024, s);
    if (n == 2) return launch_set<2>(segs, 2, fn, grid_x, 1024, s);
    return launch_set<4>(segs, n, fn, grid_x, 1024, s);
}

hipError_t launch_down_combine_iq2(const DownCombineArgs& a, hipStream_t s) {
    if (a.units == 0 || a.units > kDcMaxUnits || a.tiles == 0 || a.cols > a.units * 256 ||
        a.x2_off + a.cols > a.x_stride || (uint64_t)kDcMaxProbs * a.x_stride * 4 >= (1ull << 31))
        return hipErrorInvalidValue;
    DownCombineArgs args = a;
    void* kargs[] = {&args};
    return hipLaunchKernel(reinterpret_cast<const void*>(&down_combine_iq2_kernel), dim3(a.tiles), dim3(kDcWg), kargs,
                           0, s);
}

}  // namespace mmhip
