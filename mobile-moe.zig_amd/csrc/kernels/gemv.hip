// Decode GEMV on gfx950.
//
// Quantised weights (Q8_0, IQ2_XXS): one wave per 16-row tile. Per 32-column
// block the wave runs one v_mfma_i32_16x16x32_i8 with
//   B = 8 signed int8 weights per lane (raw qs bytes for Q8_0; two LDS table
//       reads per lane for IQ2_XXS),
//   A = the activation's two int8 digits in rows 0 (hi) and 1 (lo),
// so lanes 0..15 receive the exact integer partial sums of their row for both
// digits, scale them by d (and the IQ2_XXS sub-block scale) and the
// activation block scale, and accumulate in f32. Every weight byte is read
// exactly once, with one 128-bit load per lane per 1 KiB record unit.
//
// Waves are persistent: the grid is sized to the device and each wave walks
// (problem, tile) pairs, so one launch can stream many matrices (all experts of
// a layer) and the 32 KiB IQ2_XXS tables are copied to LDS once per workgroup.
#include "device_common.hpp"
#include "kernels.hpp"

namespace mmhip {

namespace {

constexpr int kGemvThreads = 512;
constexpr int kUnitsPerChunk = 4;

template <int FMT>
__global__ __launch_bounds__(kGemvThreads) void gemv_q_kernel(GemvArgs a) {
    __shared__ uint32_t tab[FMT == kFmtIq2 ? kIq2TableWords : 4];
    if (FMT == kFmtIq2) {
        load_iq2_tables(tab, a.tables);
        __syncthreads();
    }
    const uint32_t lane = threadIdx.x & 63;
    const uint32_t n = lane & 15, g = lane >> 4;
    const uint32_t waves_per_block = blockDim.x >> 6;
    const uint64_t total = (uint64_t)a.n_probs * a.tiles;
    const uint64_t step = (uint64_t)gridDim.x * waves_per_block;
    const bool has_a = n < 2;
    constexpr int DPU = (FMT == kFmtIq2) ? 16 : 32;  // u16 scales per unit

    for (uint64_t w = (uint64_t)blockIdx.x * waves_per_block + (threadIdx.x >> 6); w < total; w += step) {
        const uint32_t p = (uint32_t)(w / a.tiles);
        const uint32_t t = (uint32_t)(w % a.tiles);
        const uint64_t mat = a.first_mat + p;
        const uint4* R = a.recs + mat * a.rec_stride + (uint64_t)t * a.units * 64 + lane;
        const uint16_t* D = a.dvals + mat * a.d_stride + (uint64_t)t * a.units * DPU;
        const int8_t* xd = (n == 0 ? a.xh : a.xl) + (uint64_t)p * a.xq_stride + 8 * g;
        const float* xs = a.xs + (uint64_t)p * a.xs_stride;
        float acc = 0.0f;

        for (uint32_t u0 = 0; u0 < a.units; u0 += kUnitsPerChunk) {
            uint4 r[kUnitsPerChunk];
            uint32_t dw[kUnitsPerChunk];
#pragma unroll
            for (int c = 0; c < kUnitsPerChunk; ++c) {
                if (u0 + c < a.units) {
                    r[c] = R[(uint64_t)(u0 + c) * 64];
                    dw[c] = (FMT == kFmtIq2) ? (uint32_t)D[(u0 + c) * 16 + n]
                                             : reinterpret_cast<const uint32_t*>(D)[(u0 + c) * 16 + n];
                }
            }
#pragma unroll
            for (int c = 0; c < kUnitsPerChunk; ++c) {
                const uint32_t u = u0 + c;
                if (u >= a.units) break;
                if (FMT == kFmtIq2) {
                    const float dn = f16_bits_to_f32(dw[c]);
                    const uint32_t rw[4] = {r[c].x, r[c].y, r[c].z, r[c].w};
                    // Gather the four ls bits of each sub-block from the row's four lanes.
                    uint32_t mine = 0;
#pragma unroll
                    for (int s = 0; s < 8; ++s) mine |= ((rw[s >> 1] >> (15 + 16 * (s & 1))) & 1u) << (4 * s + g);
                    mine |= __shfl_xor(mine, 16, kWave);
                    mine |= __shfl_xor(mine, 32, kWave);
#pragma unroll
                    for (int s = 0; s < 8; ++s) {
                        const uint32_t rec = rw[s >> 1] >> (16 * (s & 1));
                        const long bop = iq2_b_operand(rec, tab);
                        const uint32_t blk = u * 8 + s;
                        const long aop = has_a ? *reinterpret_cast<const long*>(xd + blk * 32) : 0;
                        const v4i dv = mfma_i8(aop, bop);
                        const float ls = (float)((mine >> (4 * s)) & 15u);
                        const float cs = dn * (0.5f + ls) * 0.25f * xs[blk];
                        acc = fmaf(digits_combine(dv[0], dv[1]), cs, acc);
                    }
                } else {
                    const long b0 = (long)(((uint64_t)r[c].y << 32) | r[c].x);
                    const long b1 = (long)(((uint64_t)r[c].w << 32) | r[c].z);
                    const uint32_t blk = 2 * u;
                    const long a0 = has_a ? *reinterpret_cast<const long*>(xd + blk * 32) : 0;
                    const long a1 = has_a ? *reinterpret_cast<const long*>(xd + blk * 32 + 32) : 0;
                    const v4i d0 = mfma_i8(a0, b0);
                    const v4i d1 = mfma_i8(a1, b1);
                    const float s0 = f16_bits_to_f32(dw[c] & 0xFFFFu) * xs[blk];
                    const float s1 = f16_bits_to_f32(dw[c] >> 16) * xs[blk + 1];
                    acc = fmaf(digits_combine(d0[0], d0[1]), s0, acc);
                    acc = fmaf(digits_combine(d1[0], d1[1]), s1, acc);
                }
            }
        }
        if (lane < 16) {
            const uint32_t row = t * 16 + n;
            if (row < a.rows) a.y[(uint64_t)p * a.y_stride + row] = acc;
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

hipError_t launch_gemv_q(const GemvArgs& a, uint32_t fmt, int num_cu, hipStream_t s) {
    const uint64_t waves = (uint64_t)a.n_probs * a.tiles;
    if (waves == 0) return hipSuccess;
    const uint64_t waves_per_block = kGemvThreads / 64;
    uint64_t blocks = (waves + waves_per_block - 1) / waves_per_block;
    const uint64_t max_blocks = (uint64_t)(num_cu > 0 ? num_cu : 256) * 2;
    if (blocks > max_blocks) blocks = max_blocks;
    if (fmt == kFmtIq2)
        gemv_q_kernel<kFmtIq2><<<(unsigned)blocks, kGemvThreads, 0, s>>>(a);
    else
        gemv_q_kernel<kFmtQ8><<<(unsigned)blocks, kGemvThreads, 0, s>>>(a);
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
