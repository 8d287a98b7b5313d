// IQ2_XXS decode building blocks shared by the GEMV (gemv_iq2.hip) and the
// one-launch decode MoE layer (decode_moe.hip): activation digit planes, the
// B operands of one record unit from the LDS tables, and the arithmetic of
// one (unit, row tile) item.
#pragma once

#include "device_common.hpp"

namespace mmhip {

// Quantises 4 columns per lane (8 lanes per 32-column block, quantize_quad)
// into the chunk's digit planes: aq[(b * 2 + digit) * 32 + column].
__device__ __forceinline__ void x_store_planes(const float (&v)[4], uint32_t nblk, uint32_t b0, uint8_t* aq,
                                               float* xs) {
    uint32_t h4, l4;
    const float s = quantize_quad(v, h4, l4);
    const uint32_t b = b0 + (threadIdx.x >> 3), jq = threadIdx.x & 7;
    if (b < nblk) {
        *reinterpret_cast<uint32_t*>(aq + b * 64 + 4 * jq) = h4;
        *reinterpret_cast<uint32_t*>(aq + b * 64 + 32 + 4 * jq) = l4;
        if (jq == 0) xs[b] = s;
    }
}

// Table words of one record unit (the lane's 8 records): e[j] holds the
// entries of records 2j and 2j + 1 side by side, which is the B operand of
// the unit's j-th 16x16x64 MFMA once the hi3 signs are applied to words 1
// and 3 in place; m[s]: record s's hi3 sign pair (below).
struct RawB {
    v4i e[4];
    uint32_t m[8];
};


// Table words of the lane's 8 records (record layout in device_common.hpp):
// the 8-byte entry keyed by the record's window, whose high word still needs
// the hi3 signs, and the record's hi3 sign pair.
__device__ __forceinline__ void fetch_b(const uint4& r, const uint32_t* tab, const uint32_t* mtab, RawB& raw) {
    const uint32_t w4[4] = {r.x, r.y, r.z, r.w};
    const char* t8 = reinterpret_cast<const char*>(tab);
    const char* m8 = reinterpret_cast<const char*>(mtab);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t d = w4[k];
        // Record 2k: window at bits 3..14, hi3 at bits 15..17; record 2k + 1:
        // window at bits 18..29, hi3 at bits 0..2.
        const uint2 lo = *reinterpret_cast<const uint2*>(t8 + (d & 0x7FF8u));
        const uint2 hi = *reinterpret_cast<const uint2*>(t8 + ((d >> 15) & 0x7FF8u));
        raw.e[k] = v4i{(int)lo.x, (int)lo.y, (int)hi.x, (int)hi.y};
        raw.m[2 * k] = *reinterpret_cast<const uint32_t*>(m8 + ((d >> 13) & 0x1Cu));
        raw.m[2 * k + 1] = *reinterpret_cast<const uint32_t*>(m8 + ((d << 2) & 0x1Cu));
    }
}

// Applies the hi3 signs in place: raw.e[j] becomes the B operand of the
// unit's j-th MFMA (K order: record 2j's bytes, then record 2j + 1's; the A
// operand pairs its bytes the same way).
__device__ __forceinline__ void finish_b(RawB& raw) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        raw.e[k][1] = (int)negate_bytes((uint32_t)raw.e[k][1], raw.m[2 * k]);
        raw.e[k][3] = (int)negate_bytes((uint32_t)raw.e[k][3], raw.m[2 * k + 1]);
    }
}

// silu(x) = x / (1 + e^-x) (math.zig:38-41) with the hardware exp2 and
// reciprocal (a few ulp from the correctly rounded quotient): each workgroup
// here forms every expert's activation, so the IEEE division and expf would
// dominate its arithmetic.
__device__ __forceinline__ float silu_fast(float x) {
    return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.4426950408889634f));
}

// One item: record unit r (this lane's 16 bytes, row scale bits dbits) times
// the unit's activation digit planes aq_unit (8 blocks, x_store_planes
// layout) with block scales xs_unit. Returns lane (g, n)'s partial of row n:
// blocks g and g + 4, both digits, scaled. n = lane % 16, g = lane / 16.
__device__ __forceinline__ float iq2_item(const uint4& r, uint16_t dbits, const uint8_t* aq_unit,
                                          const float* xs_unit, const uint32_t* tab, const uint32_t* mtab,
                                          uint32_t n, uint32_t g) {
    // Sparse A row of this lane: block s_star of the unit, digit d_star.
    const uint32_t s_star = (n >> 2) + 4 * ((n >> 1) & 1u), d_star = n & 1u;
    RawB raw;
    fetch_b(r, tab, mtab, raw);
    const uint2 xw = *reinterpret_cast<const uint2*>(aq_unit + (s_star * 2 + d_star) * 32 + 8 * g);
    v4i av[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const bool lo = s_star == 2u * q, hi = s_star == 2u * q + 1;
        av[q] = v4i{(int)(lo ? xw.x : 0u), (int)(lo ? xw.y : 0u), (int)(hi ? xw.x : 0u), (int)(hi ? xw.y : 0u)};
    }
    const float xa = xs_unit[g] * 0.25f, xb4 = xs_unit[g + 4] * 0.25f;
    finish_b(raw);
    v4i acc = {0, 0, 0, 0};
#pragma unroll
    for (int q = 0; q < 4; ++q) acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(av[q], raw.e[q], acc, 0, 0, 0);
    const float sa = fmaf((float)iq2_ls_a(r), xa, xa * 0.5f);
    const float sb = fmaf((float)iq2_ls_b(r), xb4, xb4 * 0.5f);
    float v = (float)digits_combine(acc[0], acc[1]) * sa;
    v = fmaf((float)digits_combine(acc[2], acc[3]), sb, v);
    return v * f16_scale(dbits);
}

// An item's 16 row values: ((g0 + g1) + g2) + g3 of the lane partials of
// lane groups g = 0..3 (the order in which the decode GEMV sums a row's four
// lane groups), valid in lanes 0..15 (row n in lane n). permlane16_swap(v, v)
// returns v's rows (0, 0, 2, 2) and (1, 1, 3, 3); permlane32_swap(x, x)'s
// second result is x's rows (2, 3, 2, 3).
__device__ __forceinline__ float item_rows(float v) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    const auto x2 = __builtin_amdgcn_permlane32_swap(p[0], p[0], false, false);
    const auto y2 = __builtin_amdgcn_permlane32_swap(p[1], p[1], false, false);
    return ((__uint_as_float(p[0]) + __uint_as_float(p[1])) + __uint_as_float(x2[1])) + __uint_as_float(y2[1]);
}

}  // namespace mmhip
