// Batched quantised matmul (prompt prefill, qmm.matMulQ8_0's role) on gfx950.
//
// Y = X . W^T with X quantised per row to two int8 digits. Each wave owns a
// 16-row weight tile and kTokTiles tiles of 8 activation rows (tile_mm): per
// 32-column block it builds the int8 B operand once (raw Q8_0 bytes or
// IQ2_XXS LDS tables) and runs one v_mfma_i32_16x16x32_i8 per row tile with
// A rows 2j / 2j+1 = the hi / lo digits of row j.
//
// Dense mode: one matrix, rows b < batch, blockIdx.y = 32-row chunk.
// Grouped mode (MoE experts, sorted by expert): blockIdx.y = work item
// {matrix, first slot, count}; activation row of slot s = a_row[s] (or s),
// output row = s.
#include "device_common.hpp"
#include "kernels.hpp"
#include "tile_ops.hpp"

namespace mmhip {

namespace {

constexpr int kQmmThreads = 256;
constexpr int kTokTiles = kQmmTokens / 8;  // 32 rows per wave

struct QmmArgs {
    const uint4* recs;
    const uint16_t* dvals;
    uint64_t rec_stride, d_stride;
    uint32_t d_row;
    const int8_t* xh;
    const int8_t* xl;
    const float* xs;
    uint64_t xq_stride, xs_stride;
    float* y;
    uint64_t y_ld;
    uint32_t tiles, units, rows, batch;
    int out_layout;
    uint64_t mat;                 // dense mode
    const QmmWork* work;          // grouped mode when non-null
    const uint32_t* n_work;
    const uint32_t* a_row;        // grouped: activation row of each slot, or null
};

template <int FMT>
__global__ __launch_bounds__(kQmmThreads) void qmm_kernel(QmmArgs a) {
    __shared__ __align__(16) uint32_t tab[FMT == kFmtIq2 ? kIq2TableWords : 4];
    uint64_t mat = a.mat;
    uint32_t first = blockIdx.y * kQmmTokens, count = 0, col_off = 0;
    if (a.work) {
        if (blockIdx.y >= *a.n_work) return;  // whole workgroup
        const QmmWork w = a.work[blockIdx.y];
        mat = w.mat;
        first = w.slot;
        count = w.count;
        col_off = w.pad;
    } else {
        count = a.batch > first ? min(a.batch - first, kQmmTokens) : 0;
    }
    if (FMT == kFmtIq2) {
        build_iq2_tables<kQmmThreads>(tab, iq2_grid_entry());
        lds_barrier();
    }
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t n = lane & 15, g = lane >> 4;
    const uint32_t t = blockIdx.x * (kQmmThreads / 64) + (threadIdx.x >> 6);
    if (t >= a.tiles) return;
    auto act_row = [&](uint32_t j) -> uint64_t {
        const uint32_t s = first + j;
        return (a.work && a.a_row) ? a.a_row[s] : s;
    };
    ActTiles<kTokTiles> act;
#pragma unroll
    for (int tt = 0; tt < kTokTiles; ++tt) {
        const uint32_t j = tt * 8 + n / 2;
        act.a_row[tt] = j < count ? ((n & 1) ? a.xl : a.xh) + act_row(j) * a.xq_stride + 8 * g : nullptr;
        const uint32_t j0 = tt * 8 + 2 * g, j1 = j0 + 1;
        act.s0[tt] = a.xs + act_row(j0 < count ? j0 : 0) * a.xs_stride;
        act.s1[tt] = a.xs + act_row(j1 < count ? j1 : 0) * a.xs_stride;
    }
    float acc[kTokTiles][2];
    tile_mm<FMT, kTokTiles>(a.recs + mat * a.rec_stride + (uint64_t)t * a.units * 64 + lane,
                            a.dvals + mat * a.d_stride + ((uint64_t)t * 16 + n) * a.d_row, a.units, act, tab, lane,
                            acc);
    const uint32_t row = t * 16 + n;
    if (row >= a.rows) return;
#pragma unroll
    for (int tt = 0; tt < kTokTiles; ++tt) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const uint32_t j = tt * 8 + 2 * g + i;
            if (j < count) {
                const uint64_t s = first + j;
                if (a.out_layout == 0) a.y[s * a.y_ld + col_off + row] = acc[tt][i];
                else a.y[(uint64_t)row * a.y_ld + s] = acc[tt][i];
            }
        }
    }
}

QmmArgs base_args(const uint4* recs, const uint16_t* dvals, const TileGeom& g, const QuantAct& xq, float* y,
                  uint64_t y_ld) {
    QmmArgs a{};
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
    a.y_ld = y_ld;
    a.tiles = (uint32_t)g.tiles;
    a.units = (uint32_t)g.units;
    a.rows = (uint32_t)g.rows;
    return a;
}

hipError_t launch(const QmmArgs& a, uint32_t fmt, unsigned grid_y, hipStream_t s) {
    dim3 grid((unsigned)((a.tiles + 3) / 4), grid_y);
    if (fmt == kFmtIq2)
        qmm_kernel<kFmtIq2><<<grid, kQmmThreads, 0, s>>>(a);
    else
        qmm_kernel<kFmtQ8><<<grid, kQmmThreads, 0, s>>>(a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_qmm(const uint4* recs, const uint16_t* dvals, const TileGeom& g, uint64_t mat,
                      const QuantAct& xq, uint32_t batch, float* y, uint64_t y_ld, int out_layout, hipStream_t s) {
    if (batch == 0 || g.tiles == 0) return hipSuccess;
    QmmArgs a = base_args(recs, dvals, g, xq, y, y_ld);
    a.mat = mat;
    a.batch = batch;
    a.out_layout = out_layout;
    return launch(a, g.fmt, (batch + kQmmTokens - 1) / kQmmTokens, s);
}

hipError_t launch_qmm_grouped(const uint4* recs, const uint16_t* dvals, const TileGeom& g, const QuantAct& xq,
                              const uint32_t* a_row, const QmmWork* work, const uint32_t* n_work,
                              uint32_t max_work, float* y, uint64_t y_ld, hipStream_t s) {
    if (max_work == 0 || g.tiles == 0) return hipSuccess;
    QmmArgs a = base_args(recs, dvals, g, xq, y, y_ld);
    a.work = work;
    a.n_work = n_work;
    a.a_row = a_row;
    a.out_layout = 0;
    return launch(a, g.fmt, max_work, s);
}

}  // namespace mmhip
