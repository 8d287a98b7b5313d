// Per-wave pieces shared by the decode GEMV and the grouped matmul: the step
// loads of the record stream and the decode step products.
//
// Decode (one activation vector, A operand from the LDS A layout):
//   step_dot_* processes up to 8 record units of one 16-row tile. Each
//   32-column block is one v_mfma_i32_16x16x32_i8 with A rows 0/1 = the
//   vector's hi/lo digits; the integer results of four consecutive blocks are
//   gathered one per 16-lane row (gather_rows4), so every lane group scales and
//   accumulates a different block: lane (g, n) accumulates blocks with
//   index % 4 == g of row n. reduce_groups() folds the four partial sums into
//   lanes 0..15 at the end of a tile.
//
// Batched products (8 activation rows per item) live in group.hip.
#pragma once

#include "device_common.hpp"
#include "kernels.hpp"

namespace mmhip {

constexpr int kMaxUnitsPerStep = 8;

__device__ __forceinline__ float reduce_groups(float acc) {
    acc += __shfl_xor(acc, 16, kWave);
    acc += __shfl_xor(acc, 32, kWave);
    return acc;
}

// All 8 B operands of an IQ2_XXS record unit (LDS table reads).
__device__ __forceinline__ void iq2_decode_unit(const uint4& rr, const uint32_t* tab, long (&b)[8]) {
    const uint32_t w4[4] = {rr.x, rr.y, rr.z, rr.w};
#pragma unroll
    for (int s = 0; s < 8; ++s) b[s] = (s & 1) ? iq2_bop_hi(w4[s >> 1], tab) : iq2_bop_lo(w4[s >> 1], tab);
}

// One step's records (UPS units, 1 KiB apart) and the row's scale words for
// them. rec_soff / d_soff are the step's uniform byte offsets (kBufOob for a
// step past the wave's end); rec_voff = lane * 16, d_voff = the row's scale
// run. Scale runs are 16-byte aligned rows of d_row u16.
template <int FMT, int UPS>
__device__ __forceinline__ void load_step(BufRsrc rr, uint32_t rec_voff, uint32_t rec_soff, BufRsrc dr,
                                          uint32_t d_voff, uint32_t d_soff, uint4 (&r)[kMaxUnitsPerStep],
                                          uint32_t (&dw)[kMaxUnitsPerStep]) {
#pragma unroll
    for (int i = 0; i < UPS; ++i) r[i] = buf_load_b128<kCacheStream>(rr, rec_voff + i * 1024, rec_soff);
    if (FMT == kFmtIq2) {
        // Kept packed (two f16 per dword, see iq2_scale_bits): unpacking at
        // the load would make the compiler wait for the data right there.
        if (UPS == 8) {
            const uint4 q = buf_load_b128<kCacheStream>(dr, d_voff, d_soff);
            dw[0] = q.x;
            dw[1] = q.y;
            dw[2] = q.z;
            dw[3] = q.w;
        } else if (UPS == 4) {
            const uint2 q = buf_load_b64<kCacheStream>(dr, d_voff, d_soff);
            dw[0] = q.x;
            dw[1] = q.y;
        } else if (UPS == 2) {
            dw[0] = buf_load_b32<kCacheStream>(dr, d_voff, d_soff);
        } else {
#pragma unroll
            for (int i = 0; i < UPS; ++i) dw[i] = buf_load_b16<kCacheStream>(dr, d_voff + 2 * i, d_soff);
        }
    } else {
        // Q8_0: one u32 (two f16) per unit; steps of 4 or 8 units start on
        // 16-byte boundaries.
#pragma unroll
        for (int h = 0; h < UPS / 4; ++h) {
            const uint4 q = buf_load_b128<kCacheStream>(dr, d_voff + 16 * h, d_soff);
            dw[4 * h] = q.x;
            dw[4 * h + 1] = q.y;
            dw[4 * h + 2] = q.z;
            dw[4 * h + 3] = q.w;
        }
    }
}

// f16 scale bits of unit i of a decode step: steps of 2, 4 or 8 units load
// their scales packed two per dword, other step sizes one per word.
template <int UPS>
__device__ __forceinline__ uint32_t iq2_scale_bits(const uint32_t (&dw)[kMaxUnitsPerStep], int i) {
    if (UPS == 2 || UPS == 4 || UPS == 8) return (dw[i >> 1] >> (16 * (i & 1))) & 0xFFFFu;
    return dw[i];
}

// Q8_0: units in pairs (four 32-column blocks per gather); a pair is half of
// a 256-column A group. UPS is 4 or 8 and ub a multiple of 4, so steps start
// on A-group boundaries.
template <int UPS>
__device__ __forceinline__ void step_dot_q8(const uint4 (&r)[kMaxUnitsPerStep],
                                            const uint32_t (&dw)[kMaxUnitsPerStep], uint32_t ub,
                                            const int8_t* a_run, bool has_a, const float* xs_g, uint32_t g,
                                            float& acc) {
    long av[8];
#pragma unroll
    for (int i = 0; i < UPS; i += 2) {
        const bool two = i + 1 < UPS;
        const uint32_t blk0 = (ub + i) * 2;
        if ((i & 3) == 0 && has_a) lds_a_group(av, a_run, blk0 >> 3);
        const int half = (i >> 1) & 1;
        int v[4];
#pragma unroll
        for (int bb = 0; bb < 4; ++bb) {
            if (bb >= 2 && !two) {
                v[bb] = 0;
                continue;
            }
            const uint4& rr = r[i + (bb >> 1)];
            const long bop = (bb & 1) ? (long)(((uint64_t)rr.w << 32) | rr.z) : (long)(((uint64_t)rr.y << 32) | rr.x);
            const v4i dv = mfma_i8(av[4 * half + bb], bop);
            v[bb] = digits_combine(dv[0], dv[1]);
        }
        const int w = gather_rows4(v[0], v[1], v[2], v[3]);
        // lane group g scales block blk0 + g: unit i + g/2, half g&1
        const uint32_t dsel = (g >= 2) ? (two ? dw[i + 1 < UPS ? i + 1 : i] : 0u) : dw[i];
        const float d = f16_scale((dsel >> (16 * (g & 1))) & 0xFFFFu);
        const float c = (g >= 2 && !two) ? 0.0f : d * xs_g[blk0];
        acc = fmaf((float)w, c, acc);
    }
}

}  // namespace mmhip
