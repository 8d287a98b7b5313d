// Decode GEMV on gfx950.
//
// Quantised weights (Q8_0, IQ2_XXS): a workgroup owns one activation vector
// (problem) and a contiguous range of 16-row tiles. It quantises the vector
// into LDS (the A operand of every MFMA, so the separate quantisation launch
// disappears), copies the 32 KiB IQ2_XXS sign/grid tables into LDS, and each
// wave then streams its tiles' 1 KiB record units with one 128-bit load per
// lane, double-buffered so the next step's loads are in flight while the
// current one computes. Every weight byte is read exactly once.
//
// f32 / f16 weights (the router, matVecMulUnified's f32 branch): one wave
// per output row.
#include "device_common.hpp"
#include "kernels.hpp"
#include "tile_ops.hpp"

#include <cstdlib>

namespace mmhip {

namespace {

constexpr uint32_t kChunkBlocks = 256;  // 8192 columns of activation per LDS chunk (multiple of 8)

// One step's records (UPS units) and the row's scale words for them.
template <int FMT, int UPS>
__device__ __forceinline__ void load_step(const uint4* R, const uint16_t* Drow, uint32_t u_first,
                                          uint4 (&r)[kMaxUnitsPerStep], uint32_t (&dw)[kMaxUnitsPerStep]) {
#pragma unroll
    for (int i = 0; i < UPS; ++i) r[i] = R[(uint64_t)(u_first + i) * 64];
    // Scale runs are 16-byte aligned rows; vector loads where the step size allows.
    if (FMT == kFmtIq2 && (UPS == 8 || UPS == 6)) {
        const uint4 q = *reinterpret_cast<const uint4*>(Drow + u_first);
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int i = 0; i < UPS; ++i) dw[i] = (w[i >> 1] >> (16 * (i & 1))) & 0xFFFFu;
    } else if (FMT == kFmtIq2 && UPS == 4) {
        const uint2 q = *reinterpret_cast<const uint2*>(Drow + u_first);
        const uint32_t w[2] = {q.x, q.y};
#pragma unroll
        for (int i = 0; i < UPS; ++i) dw[i] = (w[i >> 1] >> (16 * (i & 1))) & 0xFFFFu;
    } else if (FMT == kFmtQ8 && (UPS == 4 || UPS == 8)) {
#pragma unroll
        for (int h = 0; h < UPS / 4; ++h) {
            const uint4 q = *reinterpret_cast<const uint4*>(Drow + 2 * (u_first + 4 * h));
            dw[4 * h] = q.x;
            dw[4 * h + 1] = q.y;
            dw[4 * h + 2] = q.z;
            dw[4 * h + 3] = q.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < UPS; ++i) dw[i] = unit_dbits<FMT>(Drow, u_first + i);
    }
}

// UPS = record units per step (compile-time); a tile's units in a K-chunk
// are a whole number of steps. WG threads per workgroup.
template <int FMT, int UPS, int WG>
__global__ __launch_bounds__(WG, (WG == 256 ? 4 : 2)) void gemv_q_kernel(GemvArgs a) {
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
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t p = blockIdx.y;
    const uint64_t mat = a.first_mat + p;
    const float* x = a.x + (uint64_t)p * a.x_stride;
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
    const uint4* rec0 = a.recs + mat * a.rec_stride + lane;
    const uint16_t* drow0 = a.dvals + mat * a.d_stride + (uint64_t)n * a.d_row;

    // Step s of a K-chunk starting at unit u_begin: tile i = s / n_sub,
    // units [u_begin + UPS * (s % n_sub), +UPS).
    uint32_t u_begin = 0;
    uint32_t n_sub = min(a.units, chunk_units) / UPS;
    auto tile_of = [&](uint32_t s) { return t_begin + wave + kWaves * (s / n_sub); };
    auto first_unit = [&](uint32_t s) { return u_begin + (s % n_sub) * UPS; };
    uint4 r[kMaxUnitsPerStep];
    uint32_t dw[kMaxUnitsPerStep];
    auto load = [&](uint32_t s) {
        const uint32_t t = tile_of(s);
        load_step<FMT, UPS>(rec0 + (uint64_t)t * a.units * 64, drow0 + (uint64_t)t * 16 * a.d_row, first_unit(s), r,
                            dw);
    };

    // The first step's weight loads go out before the prologue, so HBM
    // latency overlaps the table copy and the activation quantisation.
    uint32_t steps = my_n * n_sub;
    if (steps > 0) load(0);
    if (FMT == kFmtIq2) load_iq2_tables(tab, a.tables);

    for (uint32_t kb = 0; kb < nblk_all; kb += chunk_blk) {
        const uint32_t nb = min(chunk_blk, nblk_all - kb);
        if (kb > 0) {
            __syncthreads();  // previous chunk's LDS no longer in use
            u_begin = kb / kBlkPerUnit;
            n_sub = (nb / kBlkPerUnit) / UPS;
            steps = my_n * n_sub;
            if (steps > 0) load(0);
        }
        quantize_to_lds(x + kb * 32, a.cols > kb * 32 ? a.cols - kb * 32 : 0, nb, aq, xs);
        __syncthreads();

        float acc = 0.0f;
        for (uint32_t s = 0; s < steps; ++s) {
            if (s > 0) load(s);
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
                    float* yp = a.y + (uint64_t)p * a.y_stride + row;
                    *yp = (kb == 0) ? tot : *yp + tot;
                }
            }
        }
    }
}

// f32 / f16 weights: one wave per output row.
template <typename WT>
__global__ __launch_bounds__(256) void gemv_float_kernel(const WT* __restrict__ w, uint64_t mat_stride,
                                                         const float* __restrict__ x, uint64_t x_stride,
                                                         float* __restrict__ y, uint64_t y_stride,
                                                         uint32_t n_mats, uint32_t rows, uint32_t cols) {
    const uint32_t lane = threadIdx.x & 63;
    const uint64_t wid = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    if (wid >= (uint64_t)n_mats * rows) return;
    const uint32_t m = (uint32_t)(wid / rows), r = (uint32_t)(wid % rows);
    const WT* wr = w + m * mat_stride + (uint64_t)r * cols;
    const float* xv = x + m * x_stride;
    float acc = 0.0f;
    for (uint32_t c = lane; c < cols; c += 64) {
        float wv;
        if constexpr (sizeof(WT) == 2) wv = f16_bits_to_f32(wr[c]);
        else wv = wr[c];
        acc = fmaf(wv, xv[c], acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) y[m * y_stride + r] = acc;
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
static void launch_ups(int ups, dim3 grid, size_t lds, hipStream_t s, const GemvArgs& a) {
    switch (ups) {
        case 1: gemv_q_kernel<FMT, 1, WG><<<grid, WG, lds, s>>>(a); break;
        case 2: gemv_q_kernel<FMT, 2, WG><<<grid, WG, lds, s>>>(a); break;
        case 3: gemv_q_kernel<FMT, 3, WG><<<grid, WG, lds, s>>>(a); break;
        case 4: gemv_q_kernel<FMT, 4, WG><<<grid, WG, lds, s>>>(a); break;
        case 5: gemv_q_kernel<FMT, 5, WG><<<grid, WG, lds, s>>>(a); break;
        case 6: gemv_q_kernel<FMT, 6, WG><<<grid, WG, lds, s>>>(a); break;
        case 7: gemv_q_kernel<FMT, 7, WG><<<grid, WG, lds, s>>>(a); break;
        default: gemv_q_kernel<FMT, 8, WG><<<grid, WG, lds, s>>>(a); break;
    }
}

static int env_int(const char* name, int dflt) {
    const char* e = getenv(name);
    return e ? atoi(e) : dflt;
}

hipError_t launch_gemv_q(const GemvArgs& a_in, uint32_t fmt, int num_cu, hipStream_t s) {
    if (a_in.n_probs == 0 || a_in.tiles == 0) return hipSuccess;
    GemvArgs a = a_in;
    // Tuning knobs (defaults measured on MI355X): MMHIP_GEMV_WG threads per
    // workgroup (256 | 512), MMHIP_GEMV_MAX_UPS caps record units per step,
    // MMHIP_GEMV_WG_PER_CU the workgroups per CU the grid aims for.
    static const int wg = env_int("MMHIP_GEMV_WG", 256) == 512 ? 512 : 256;
    static const int cap_env = env_int("MMHIP_GEMV_MAX_UPS", 0);
    // IQ2_XXS steps above 4 units exceed 128 VGPRs (4 waves per SIMD) and spill.
    const int cap = cap_env > 0 ? cap_env : (fmt == kFmtIq2 ? 4 : 8);
    static const int wg_per_cu = env_int("MMHIP_GEMV_WG_PER_CU", 4);
    const uint32_t waves = wg / 64;
    const uint64_t total_tiles = (uint64_t)a.n_probs * a.tiles;
    const uint64_t target_wgs = (uint64_t)(num_cu > 0 ? num_cu : 256) * (wg_per_cu > 0 ? wg_per_cu : 4);
    uint64_t tpw = (total_tiles + target_wgs - 1) / target_wgs;  // tiles per WG
    tpw = (tpw + waves - 1) / waves * waves;
    if (tpw < waves) tpw = waves;
    if (tpw > a.tiles) tpw = (a.tiles + waves - 1) / waves * waves;
    a.tiles_per_wg = (uint32_t)tpw;
    dim3 grid((unsigned)((a.tiles + tpw - 1) / tpw), a.n_probs);
    const size_t lds = gemv_q_lds_bytes(fmt, a.units);
    int ups = pick_ups(fmt, a.units);
    if (ups == 0) return hipErrorInvalidValue;
    while (ups > cap && ups % 2 == 0 && (fmt == kFmtIq2 || ups > 4)) ups /= 2;
    if (fmt == kFmtIq2) {
        if (wg == 512) launch_ups<kFmtIq2, 512>(ups, grid, lds, s, a);
        else launch_ups<kFmtIq2, 256>(ups, grid, lds, s, a);
    } else {
        if (wg == 512) launch_ups<kFmtQ8, 512>(ups, grid, lds, s, a);
        else launch_ups<kFmtQ8, 256>(ups, grid, lds, s, a);
    }
    return hipGetLastError();
}

hipError_t launch_gemv_float(const void* w, uint32_t type, uint64_t mat_stride, const float* x,
                             uint64_t x_stride, float* y, uint64_t y_stride, uint32_t n_mats,
                             uint32_t rows, uint32_t cols, hipStream_t s) {
    const uint64_t waves = (uint64_t)n_mats * rows;
    if (waves == 0) return hipSuccess;
    const unsigned blocks = (unsigned)((waves * 64 + 255) / 256);
    if (type == 0)
        gemv_float_kernel<float><<<blocks, 256, 0, s>>>((const float*)w, mat_stride, x, x_stride, y, y_stride,
                                                        n_mats, rows, cols);
    else
        gemv_float_kernel<uint16_t><<<blocks, 256, 0, s>>>((const uint16_t*)w, mat_stride, x, x_stride, y,
                                                           y_stride, n_mats, rows, cols);
    return hipGetLastError();
}

}  // namespace mmhip
