// Batched quantised matmul (prompt prefill, qmm.matMulQ8_0's role) on gfx950.
//
// Y = X . W^T with X quantised per token to two int8 digits. Each wave owns a
// 16-row weight tile and kTokTiles tiles of 8 tokens; per 32-column block it
// builds the int8 B operand once (raw Q8_0 bytes or IQ2_XXS LDS tables) and
// runs one v_mfma_i32_16x16x32_i8 per token tile with A rows 2j / 2j+1 = the
// hi / lo digits of token j. Lane (q, n) then holds, for weight row n, the
// integer partial sums of tokens 2q and 2q+1 of the tile.
#include "device_common.hpp"
#include "kernels.hpp"

namespace mmhip {

namespace {

constexpr int kQmmThreads = 256;
constexpr int kTokTiles = 4;  // 32 tokens per wave

struct QmmArgs {
    const uint4* recs;
    const uint16_t* dvals;
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
        load_iq2_tables(tab, a.tables);
        __syncthreads();
    }
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t n = lane & 15, g = lane >> 4;
    const uint32_t t = blockIdx.x * (kQmmThreads / 64) + (threadIdx.x >> 6);
    if (t >= a.tiles) return;
    const uint32_t tok_base = blockIdx.y * (kTokTiles * 8);
    constexpr int DPU = (FMT == kFmtIq2) ? 16 : 32;
    const uint4* R = a.recs + (uint64_t)t * a.units * 64 + lane;
    const uint16_t* D = a.dvals + (uint64_t)t * a.units * DPU;

    // A operand source of this lane for each token tile: token m/2, digit m&1.
    const int8_t* arow[kTokTiles];
    bool aval[kTokTiles];
    const float* xs0[kTokTiles];
    const float* xs1[kTokTiles];
    bool v0[kTokTiles], v1[kTokTiles];
#pragma unroll
    for (int tt = 0; tt < kTokTiles; ++tt) {
        const uint32_t tok = tok_base + tt * 8 + n / 2;
        aval[tt] = tok < a.batch;
        arow[tt] = ((n & 1) ? a.xl : a.xh) + (uint64_t)(aval[tt] ? tok : 0) * a.xq_stride + 8 * g;
        const uint32_t t0 = tok_base + tt * 8 + 2 * g, t1 = t0 + 1;
        v0[tt] = t0 < a.batch;
        v1[tt] = t1 < a.batch;
        xs0[tt] = a.xs + (uint64_t)(v0[tt] ? t0 : 0) * a.xs_stride;
        xs1[tt] = a.xs + (uint64_t)(v1[tt] ? t1 : 0) * a.xs_stride;
    }
    float acc[kTokTiles][2];
#pragma unroll
    for (int tt = 0; tt < kTokTiles; ++tt) acc[tt][0] = acc[tt][1] = 0.0f;

    for (uint32_t u = 0; u < a.units; ++u) {
        const uint4 r = R[(uint64_t)u * 64];
        if (FMT == kFmtIq2) {
            const float dn = f16_bits_to_f32(D[u * 16 + n]);
            const uint32_t rw[4] = {r.x, r.y, r.z, r.w};
            uint32_t mine = 0;
#pragma unroll
            for (int s = 0; s < 8; ++s) mine |= ((rw[s >> 1] >> (15 + 16 * (s & 1))) & 1u) << (4 * s + g);
            mine |= __shfl_xor(mine, 16, kWave);
            mine |= __shfl_xor(mine, 32, kWave);
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                const long bop = iq2_b_operand(rw[s >> 1] >> (16 * (s & 1)), tab);
                const uint32_t blk = u * 8 + s;
                const float cw = dn * (0.5f + (float)((mine >> (4 * s)) & 15u)) * 0.25f;
#pragma unroll
                for (int tt = 0; tt < kTokTiles; ++tt) {
                    const long aop = aval[tt] ? *reinterpret_cast<const long*>(arow[tt] + blk * 32) : 0;
                    const v4i dv = mfma_i8(aop, bop);
                    acc[tt][0] = fmaf(digits_combine(dv[0], dv[1]), cw * xs0[tt][blk], acc[tt][0]);
                    acc[tt][1] = fmaf(digits_combine(dv[2], dv[3]), cw * xs1[tt][blk], acc[tt][1]);
                }
            }
        } else {
            const uint32_t dd = reinterpret_cast<const uint32_t*>(D)[u * 16 + n];
            const long bops[2] = {(long)(((uint64_t)r.y << 32) | r.x), (long)(((uint64_t)r.w << 32) | r.z)};
            const float cws[2] = {f16_bits_to_f32(dd & 0xFFFFu), f16_bits_to_f32(dd >> 16)};
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                const uint32_t blk = 2 * u + b;
#pragma unroll
                for (int tt = 0; tt < kTokTiles; ++tt) {
                    const long aop = aval[tt] ? *reinterpret_cast<const long*>(arow[tt] + blk * 32) : 0;
                    const v4i dv = mfma_i8(aop, bops[b]);
                    acc[tt][0] = fmaf(digits_combine(dv[0], dv[1]), cws[b] * xs0[tt][blk], acc[tt][0]);
                    acc[tt][1] = fmaf(digits_combine(dv[2], dv[3]), cws[b] * xs1[tt][blk], acc[tt][1]);
                }
            }
        }
    }
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
