// Decode GEMV on gfx950.
//
// Quantised weights (Q8_0, IQ2_XXS): a workgroup owns one activation vector
// (problem) and a contiguous range of 16-row tiles. It quantises the vector
// into LDS (the A operand of every MFMA, so the separate quantisation launch
// disappears), builds the 32 KiB IQ2_XXS sign/grid tables in LDS from the
// 2 KiB grid, and each wave then streams its tiles' 1 KiB record units with one 128-bit load per
// lane, through a ring of three register buffers so the next two steps'
// loads are in flight while the current one computes. Every weight byte is read exactly once.
//
// f32 / f16 weights (the router, matVecMulUnified's f32 branch): one
// workgroup per output row.
#include "device_common.hpp"
#include "kernels.hpp"
#include "tile_ops.hpp"

#include <cstdlib>
#include <map>
#include <mutex>

namespace mmhip {

namespace {

constexpr uint32_t kChunkBlocks = 256;  // 8192 columns of activation per LDS chunk (multiple of 8)

// UPS = record units per step (compile-time); a tile's units in a K-chunk
// are a whole number of steps. WG threads per workgroup.
//
// Loads: every weight, scale and activation load goes through a buffer
// resource and is issued unconditionally (out-of-range offsets for steps past
// the wave's end), so each wait covers exactly the loads it needs. The
// prologue issues the grid entry and the activation loads of all waves first,
// then the first three steps' weights, and only then waits on the small
// loads.
// A ring of three register buffers keeps the next two steps' loads in flight
// while a step computes.
template <int FMT, int UPS, int WG>
__global__ __launch_bounds__(WG, (WG == 256 ? 3 : 2)) void gemv_q_kernel(GemvArgs a) {
    constexpr uint32_t kWaves = WG / 64;
    // Static LDS for the tables (known address: table offsets fold into the
    // ds_read immediates); dynamic LDS for the activation chunk.
    __shared__ __align__(16) uint32_t tab[FMT == kFmtIq2 ? kIq2TableWords : 4];
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr uint32_t kBlkPerUnit = (FMT == kFmtIq2) ? 8 : 2;
    const uint32_t nblk_all = a.units * kBlkPerUnit;
    const uint32_t chunk_blk = nblk_all < kChunkBlocks ? nblk_all : kChunkBlocks;
    const uint32_t chunk_units = chunk_blk / kBlkPerUnit;
    int8_t* aq = reinterpret_cast<int8_t*>(smem);
    float* xs = reinterpret_cast<float*>(smem + ((chunk_blk + 7) / 8) * kAGroupBytes);

    const uint32_t lane = threadIdx.x & 63;
    const uint32_t n = lane & 15, g = lane >> 4;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t p = blockIdx.y;
    if (a.n_active && p >= *a.n_active) return;  // whole workgroup: problem not in this call's list
    uint64_t mat = a.first_mat + p, x_row = p, y_row = p;
    if (a.probs) {
        const uint4 d = a.probs[p];
        mat = d.x;
        x_row = d.y;
        y_row = d.z;
    }
    const float* x = a.x + x_row * a.x_stride;
    float* const y_base = a.y + y_row * a.y_stride;
    const bool silu_mul = a.silu_mul != 0;
    const uint32_t t_begin = blockIdx.x * a.tiles_per_wg;
    // this wave's tiles: t_begin + wave + kWaves * i, i < my_n
    uint32_t my_n = 0;
    if (t_begin + wave < a.tiles) {
        const uint32_t t_end = min(a.tiles, t_begin + a.tiles_per_wg);
        my_n = (t_end - (t_begin + wave) + kWaves - 1) / kWaves;
    }
    const bool has_a = n < 2;
    const int8_t* a_run = aq + (n & 1) * 4 * kARun + g * kARun;  // used by lanes n < 2 only
    const float* xs_g = xs + g;
    const BufRsrc rec_r = make_rsrc(a.recs + mat * a.rec_stride, (uint32_t)(a.rec_stride * 16));
    const BufRsrc d_r = make_rsrc(a.dvals + mat * a.d_stride, (uint32_t)(a.d_stride * 2));
    const uint32_t rec_voff = lane * 16;
    const uint32_t d_voff = n * a.d_row * 2;

    // Step s of a K-chunk starting at unit u_begin: tile i = s / n_sub,
    // units [u_begin + UPS * (s % n_sub), +UPS).
    uint32_t u_begin = 0;
    uint32_t n_sub = min(a.units, chunk_units) / UPS;
    auto tile_of = [&](uint32_t s) { return t_begin + wave + kWaves * (s / n_sub); };
    auto first_unit = [&](uint32_t s) { return u_begin + (s % n_sub) * UPS; };
    uint32_t steps = my_n * n_sub;
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
    float acc = 0.0f;
    uint32_t kb = 0;
    // Computes step s from (r, dw); writes the tile's row sums after its last step.
    auto compute = [&](uint32_t s, const uint4 (&r)[kMaxUnitsPerStep], const uint32_t (&dw)[kMaxUnitsPerStep]) {
        const uint32_t ub = first_unit(s) - u_begin;  // unit index within the LDS chunk
        if (FMT == kFmtIq2)
            step_dot_iq2<UPS>(r, dw, ub, a_run, has_a, xs_g, tab, acc);
        else
            step_dot_q8<UPS>(r, dw, ub, a_run, has_a, xs_g, g, acc);
        if (s % n_sub == n_sub - 1) {
            const float tot = reduce_groups(acc);
            acc = 0.0f;
            const uint32_t row = tile_of(s) * 16 + n;
            if (lane < 16 && row < a.rows) {
                float* yp = y_base + row;
                *yp = (kb == 0) ? tot : *yp + tot;
            }
        }
    };

    {
        // Prologue of the first chunk (two activation passes cover 32 * WG / 4
        // columns; longer chunks quantise the rest after the weight loads).
        const uint32_t nb = chunk_blk;
        const uint32_t xb = min(a.cols, chunk_blk * 32) * 4;
        const BufRsrc x_r = make_rsrc(x, xb);
        const BufRsrc u_r = make_rsrc(x + a.x2_off, silu_mul ? xb : 0);  // zero-size: loads read 0
        uint64_t gv = 0;
        if (FMT == kFmtIq2) gv = iq2_grid_entry();
        float xv0[4], xv1[4], uv0[4], uv1[4];
        x_pass_load(x_r, 0, xv0);
        x_pass_load(x_r, WG / 8, xv1);
        x_pass_load(u_r, 0, uv0);
        x_pass_load(u_r, WG / 8, uv1);
        // A CU serves its waves' loads in issue order: the barrier (no memory
        // fence, no wait) puts every wave's small loads ahead of the weights.
        __builtin_amdgcn_s_barrier();
        load(0, r0, d0);
        load(1, r1, d1);
        load(2, r2, d2);
        if (FMT == kFmtIq2) build_iq2_tables<WG>(tab, gv);
        if (silu_mul) {
            silu_mul4(xv0, uv0);
            silu_mul4(xv1, uv1);
        }
        x_pass_store(xv0, nb, 0, aq, xs);
        x_pass_store(xv1, nb, WG / 8, aq, xs);
        for (uint32_t b0 = 2 * (WG / 8); b0 < nb; b0 += WG / 8) {
            float v[4], u[4];
            x_pass_load(x_r, b0, v);
            x_pass_load(u_r, b0, u);
            if (silu_mul) silu_mul4(v, u);
            x_pass_store(v, nb, b0, aq, xs);
        }
    }
    for (;;) {
        lds_barrier();
        for (uint32_t s = 0; s < steps; s += 3) {
            compute(s, r0, d0);
            load(s + 3, r0, d0);
            if (s + 1 < steps) compute(s + 1, r1, d1);
            load(s + 4, r1, d1);
            if (s + 2 < steps) compute(s + 2, r2, d2);
            load(s + 5, r2, d2);
        }
        kb += chunk_blk;
        if (kb >= nblk_all) break;
        // Next K-chunk (activations longer than one LDS chunk).
        const uint32_t nb = min(chunk_blk, nblk_all - kb);
        lds_barrier();  // previous chunk's LDS no longer in use
        u_begin = kb / kBlkPerUnit;
        n_sub = (nb / kBlkPerUnit) / UPS;
        steps = my_n * n_sub;
        load(0, r0, d0);
        load(1, r1, d1);
        load(2, r2, d2);
        const uint32_t c0 = kb * 32;
        const uint32_t cb = (a.cols > c0 ? min(a.cols - c0, nb * 32) : 0) * 4;
        quantize_to_lds<WG>(make_rsrc(x + c0, cb), make_rsrc(x + a.x2_off + c0, silu_mul ? cb : 0), silu_mul, nb, aq,
                            xs);
    }
}

// f32 / f16 weights: one 256-thread workgroup per output row. Each pass
// covers 2048 columns (8 per thread) with all of a thread's loads in flight
// together; out-of-range columns read as zero through the buffer resources.
constexpr int kFloatThreads = 256;
template <typename WT>
__global__ __launch_bounds__(kFloatThreads) void gemv_float_kernel(const WT* __restrict__ w, uint64_t mat_stride,
                                                                   const float* __restrict__ x, uint64_t x_stride,
                                                                   float* __restrict__ y, uint64_t y_stride,
                                                                   uint32_t rows, uint32_t cols) {
    __shared__ float part[kFloatThreads / 64];
    const uint32_t m = blockIdx.y, r = blockIdx.x;
    const BufRsrc wr = make_rsrc(w + m * mat_stride + (uint64_t)r * cols, cols * (uint32_t)sizeof(WT));
    const BufRsrc xr = make_rsrc(x + m * x_stride, cols * 4);
    float acc = 0.0f;
    for (uint32_t c0 = 0; c0 < cols; c0 += kFloatThreads * 8) {
        const uint32_t c = c0 + threadIdx.x * 4;
        float wv[8], xv[8];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t cc = c + h * kFloatThreads * 4;
#pragma unroll
            for (int e = 0; e < 4; ++e) xv[4 * h + e] = __uint_as_float(buf_load_b32(xr, (cc + e) * 4, 0));
            if constexpr (sizeof(WT) == 2) {
#pragma unroll
                for (int e = 0; e < 4; ++e) wv[4 * h + e] = f16_bits_to_f32(buf_load_b16(wr, (cc + e) * 2, 0));
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) wv[4 * h + e] = __uint_as_float(buf_load_b32(wr, (cc + e) * 4, 0));
            }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) acc = fmaf(wv[e], xv[e], acc);
    }
    acc = wave_sum(acc);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        float t = 0.0f;
#pragma unroll
        for (int i = 0; i < kFloatThreads / 64; ++i) t += part[i];
        y[m * y_stride + r] = t;
    }
}

}  // namespace

size_t gemv_q_lds_bytes(uint32_t fmt, uint32_t units) {
    const uint32_t nblk = units * (fmt == kFmtIq2 ? 8 : 2);
    const uint32_t chunk = nblk < kChunkBlocks ? nblk : kChunkBlocks;
    return (size_t)((chunk + 7) / 8) * kAGroupBytes + (size_t)chunk * 4;  // tables are static LDS
}

// Units per step: a divisor of both the tile's unit count and the LDS
// chunk's, at most kMaxUnitsPerStep. Q8_0 tiles hold a multiple of 4 units
// (256-column A groups), and Q8_0 steps are 4 or 8 units.
static int pick_ups(uint32_t fmt, uint32_t units) {
    const uint32_t chunk_units = min(units, (uint32_t)(kChunkBlocks / (fmt == kFmtIq2 ? 8 : 2)));
    uint32_t a = units, b = chunk_units;
    while (b) {
        const uint32_t t = a % b;
        a = b;
        b = t;
    }
    const uint32_t common = a;
    if (fmt == kFmtIq2) {
        for (int u = kMaxUnitsPerStep; u >= 1; --u)
            if (common % u == 0) return u;
        return 1;
    }
    if (common % 8 == 0) return 8;
    if (common % 4 == 0) return 4;
    return 0;
}

template <int FMT, int WG>
static const void* kernel_for(int ups) {
    switch (ups) {
        case 1: return reinterpret_cast<const void*>(&gemv_q_kernel<FMT, 1, WG>);
        case 2: return reinterpret_cast<const void*>(&gemv_q_kernel<FMT, 2, WG>);
        case 3: return reinterpret_cast<const void*>(&gemv_q_kernel<FMT, 3, WG>);
        case 4: return reinterpret_cast<const void*>(&gemv_q_kernel<FMT, 4, WG>);
        case 5: return reinterpret_cast<const void*>(&gemv_q_kernel<FMT, 5, WG>);
        case 6: return reinterpret_cast<const void*>(&gemv_q_kernel<FMT, 6, WG>);
        case 7: return reinterpret_cast<const void*>(&gemv_q_kernel<FMT, 7, WG>);
        default: return reinterpret_cast<const void*>(&gemv_q_kernel<FMT, 8, WG>);
    }
}

static int env_int(const char* name, int dflt) {
    const char* e = getenv(name);
    return e ? atoi(e) : dflt;
}

// Resident workgroups per CU of one kernel instance (register and LDS
// limited), cached per (kernel, LDS bytes).
static int resident_per_cu(const void* fn, int wg, size_t lds) {
    static std::mutex mu;
    static std::map<std::pair<const void*, size_t>, int> cache;
    std::lock_guard<std::mutex> lock(mu);
    auto key = std::make_pair(fn, lds);
    auto it = cache.find(key);
    if (it != cache.end()) return it->second;
    int nb = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, fn, wg, lds) != hipSuccess || nb <= 0) nb = 1;
    cache[key] = nb;
    return nb;
}

hipError_t launch_gemv_q(const GemvArgs& a_in, uint32_t fmt, int num_cu, hipStream_t s) {
    if (a_in.n_probs == 0 || a_in.tiles == 0) return hipSuccess;
    GemvArgs a = a_in;
    // Tuning knobs (defaults measured on MI355X): MMHIP_GEMV_WG threads per
    // workgroup (256 | 512), MMHIP_GEMV_MAX_UPS caps record units per step,
    // MMHIP_GEMV_WG_PER_CU overrides the resident workgroups per CU that the
    // grid is sized for (default: the occupancy the kernel reaches).
    static const int wg = env_int("MMHIP_GEMV_WG", 256) == 512 ? 512 : 256;
    static const int cap_env = env_int("MMHIP_GEMV_MAX_UPS", 0);
    // Steps above 4 units exceed the register budget of 3 waves per SIMD
    // (168 VGPRs with two record buffers) and spill.
    const int cap = cap_env > 0 ? cap_env : 4;
    static const int wg_per_cu_env = env_int("MMHIP_GEMV_WG_PER_CU", 0);
    int ups = pick_ups(fmt, a.units);
    if (ups == 0) return hipErrorInvalidValue;
    while (ups > cap && ups % 2 == 0 && (fmt == kFmtIq2 || ups > 4)) ups /= 2;
    const void* fn = fmt == kFmtIq2 ? (wg == 512 ? kernel_for<kFmtIq2, 512>(ups) : kernel_for<kFmtIq2, 256>(ups))
                                    : (wg == 512 ? kernel_for<kFmtQ8, 512>(ups) : kernel_for<kFmtQ8, 256>(ups));
    const size_t lds = gemv_q_lds_bytes(fmt, a.units);
    const int wg_per_cu = wg_per_cu_env > 0 ? wg_per_cu_env : resident_per_cu(fn, wg, lds);
    const uint32_t waves = wg / 64;
    const uint64_t total_tiles = (uint64_t)a.n_probs * a.tiles;
    const uint64_t target_wgs = (uint64_t)(num_cu > 0 ? num_cu : 256) * wg_per_cu;
    uint64_t tpw = (total_tiles + target_wgs - 1) / target_wgs;  // tiles per WG
    tpw = (tpw + waves - 1) / waves * waves;
    if (tpw < waves) tpw = waves;
    if (tpw > a.tiles) tpw = (a.tiles + waves - 1) / waves * waves;
    a.tiles_per_wg = (uint32_t)tpw;
    dim3 grid((unsigned)((a.tiles + tpw - 1) / tpw), a.n_probs);
    void* args[] = {&a};
    return hipLaunchKernel(fn, grid, dim3(wg), args, lds, s);
}

hipError_t launch_gemv_float(const void* w, uint32_t type, uint64_t mat_stride, const float* x,
                             uint64_t x_stride, float* y, uint64_t y_stride, uint32_t n_mats,
                             uint32_t rows, uint32_t cols, hipStream_t s) {
    if ((uint64_t)n_mats * rows == 0) return hipSuccess;
    const dim3 grid(rows, n_mats);
    if (type == 0)
        gemv_float_kernel<float><<<grid, kFloatThreads, 0, s>>>((const float*)w, mat_stride, x, x_stride, y, y_stride,
                                                               rows, cols);
    else
        gemv_float_kernel<uint16_t><<<grid, kFloatThreads, 0, s>>>((const uint16_t*)w, mat_stride, x, x_stride, y,
                                                                  y_stride, rows, cols);
    return hipGetLastError();
}

}  // namespace mmhip
