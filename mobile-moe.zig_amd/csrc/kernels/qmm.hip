// Batched quantised matmul (prompt prefill, qmm.matMulQ8_0's role) on gfx950.
//
// Y = X . W^T with X quantised per token to two int8 digits. Each wave owns a
// 16-row weight tile and kTokTiles tiles of 8 tokens (tile_mm): per 32-column
// block it builds the int8 B operand once (raw Q8_0 bytes or IQ2_XXS LDS
// tables) and runs one v_mfma_i32_16x16x32_i8 per token tile with A rows
// 2j / 2j+1 = the hi / lo digits of token j.
#include "device_common.hpp"
#include "kernels.hpp"
#include "tile_ops.hpp"

namespace mmhip {

namespace {

constexpr int kQmmThreads = 256;
constexpr int kTokTiles = 4;  // 32 tokens per wave

struct QmmArgs {
    const uint4* recs;
    const uint16_t* dvals;
    uint32_t d_row;
    const int8_t* xh;
    const int8_t* xl;
    const float* xs;
    uint64_t xq_stride, xs_stride;
    float* y;
    uint64_t y_ld;
    const uint32_t* tables;
    uint32_t tiles, units, rows, batch;
    int out_layout;
};

template <int FMT>
__global__ __launch_bounds__(kQmmThreads) void qmm_kernel(QmmArgs a) {
    __shared__ uint32_t tab[FMT == kFmtIq2 ? kIq2TableWords : 4];
    if (FMT == kFmtIq2) {
        build_iq2_tables<kQmmThreads>(tab, iq2_grid_entry());
        __syncthreads();
    }
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t n = lane & 15, g = lane >> 4;
    const uint32_t t = blockIdx.x * (kQmmThreads / 64) + (threadIdx.x >> 6);
    if (t >= a.tiles) return;
    const uint32_t tok_base = blockIdx.y * (kTokTiles * 8);
    ActTiles<kTokTiles> act;
#pragma unroll
    for (int tt = 0; tt < kTokTiles; ++tt) {
        const uint32_t tok = tok_base + tt * 8 + n / 2;
        act.a_row[tt] = tok < a.batch ? ((n & 1) ? a.xl : a.xh) + (uint64_t)tok * a.xq_stride + 8 * g : nullptr;
        const uint32_t t0 = tok_base + tt * 8 + 2 * g, t1 = t0 + 1;
        act.s0[tt] = a.xs + (uint64_t)(t0 < a.batch ? t0 : 0) * a.xs_stride;
        act.s1[tt] = a.xs + (uint64_t)(t1 < a.batch ? t1 : 0) * a.xs_stride;
    }
    float acc[kTokTiles][2];
    tile_mm<FMT, kTokTiles>(a.recs + (uint64_t)t * a.units * 64 + lane,
                            a.dvals + ((uint64_t)t * 16 + n) * a.d_row, a.units, act, tab, lane, acc);
    const uint32_t row = t * 16 + n;
    if (row >= a.rows) return;
#pragma unroll
    for (int tt = 0; tt < kTokTiles; ++tt) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t tok = tok_base + tt * 8 + 2 * g + i;
            if (tok < a.batch) {
                if (a.out_layout == 0) a.y[(uint64_t)tok * a.y_ld + row] = acc[tt][i];
                else a.y[(uint64_t)row * a.y_ld + tok] = acc[tt][i];
            }
        }
    }
}

}  // namespace

hipError_t launch_qmm(const uint4* recs, const uint16_t* dvals, const TileGeom& g, uint64_t mat,
                      const QuantAct& xq, uint32_t batch, float* y, uint64_t y_ld, int out_layout,
                      const uint32_t* tables, hipStream_t s) {
    if (batch == 0 || g.tiles == 0) return hipSuccess;
    QmmArgs a;
    a.recs = recs + mat * g.rec_stride;
    a.dvals = dvals + mat * g.d_stride;
    a.d_row = (uint32_t)g.d_row;
    a.xh = xq.hi;
    a.xl = xq.lo;
    a.xs = xq.scale;
    a.xq_stride = xq.stride;
    a.xs_stride = xq.scale_stride;
    a.y = y;
    a.y_ld = y_ld;
    a.tables = tables;
    a.tiles = (uint32_t)g.tiles;
    a.units = (uint32_t)g.units;
    a.rows = (uint32_t)g.rows;
    a.batch = batch;
    a.out_layout = out_layout;
    dim3 grid((unsigned)((g.tiles + 3) / 4), (unsigned)((batch + kTokTiles * 8 - 1) / (kTokTiles * 8)));
    if (g.fmt == kFmtIq2)
        qmm_kernel<kFmtIq2><<<grid, kQmmThreads, 0, s>>>(a);
    else
        qmm_kernel<kFmtQ8><<<grid, kQmmThreads, 0, s>>>(a);
    return hipGetLastError();
}

}  // namespace mmhip
