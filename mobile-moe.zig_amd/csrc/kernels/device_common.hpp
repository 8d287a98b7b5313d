// Device-side building blocks shared by the gfx950 kernels.
//
// Tile layouts (built once at upload by repack.hip; same bytes per block as
// GGUF, only reordered):
//
//   A "row tile" is 16 consecutive output rows. For each row tile the kernels
//   read one 1 KiB record unit per 256 (IQ2_XXS) or 64 (Q8_0) input columns:
//   64 lanes x 16 B, one coalesced 128-bit load per lane. Lane l serves output
//   row n = l % 16 and column group g = l / 16 (8 consecutive columns of each
//   32-column block), which is exactly the B-operand layout of
//   v_mfma_i32_16x16x32_i8 (B[k][n], k = 8g..8g+7 in lane 16g+n).
//
//   IQ2_XXS unit (one 256-column superblock of 16 rows, 1056 B = 16 x 66 B):
//     recs: lane l holds 8 records (u16), one per 32-column sub-block s.
//       record = b012 | P<<3 | idx<<4 | hi3<<12 | lsbit<<15
//         idx    grid index of group g (byte g of the first u32 of sub-block s)
//         code   7-bit sign code of group g; b012 = code bits 0..2,
//                hi3 = code bits 4..6, P = parity of code bits 0..3
//         lsbit  bit g of the sub-block's 4-bit scale ls
//       (15 information bits of the raw format + 1 of the 4 ls bits; the four
//       lanes of a row together carry the whole ls.)
//     d:    16 x f16, one per row.
//   Signed int8 weights come from two 16 KiB LDS tables indexed straight from
//   the record: LO[(rec & 0xFFF)] (columns 0..3 of the group, signs b0..b3
//   with b3 = P ^ parity(b012)) and HI[(rec >> 3) & 0xFFF] (columns 4..7,
//   signs hi3 and bit 7 = P ^ parity(hi3), i.e. the ksigns parity bit).
//
//   Q8_0 unit (two 32-column blocks of 16 rows, 1088 B = 32 x 34 B):
//     recs: lane l holds qs[8g..8g+7] of block 2u then of block 2u+1.
//     d:    16 x (f16 d(2u), f16 d(2u+1)).
//
// Activations are quantised per 32-column block to 16-bit fixed point split in
// two int8 digits (x ~= s * (256 * hi + lo)), so one int8 MFMA over a 32-column
// block yields exact integer partial sums for both digits.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mmhip {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr int kTileRows = 16;
constexpr int kIq2UnitCols = 256;
constexpr int kQ8UnitCols = 64;
constexpr float kDigitMax = 32512.0f;  // 127 * 256: hi digit stays in [-127, 127]
constexpr int kIq2TableWords = 8192;   // LO[4096] then HI[4096], u32 each

// IEEE binary16 bits -> binary32 (dequant.zig:19-47 semantics: exact,
// subnormals normalised, Inf/NaN payload kept). Independent of the device's
// f16 denormal mode: subnormals are m * 2^-24, computed exactly in f32.
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    uint32_t s = (h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    if (e == 0) return __uint_as_float(s | __float_as_uint((float)m * 0x1p-24f));
    uint32_t bits = (e == 31u) ? (s | 0x7F800000u | (m << 13)) : (s | ((e + 112u) << 23) | (m << 13));
    return __uint_as_float(bits);
}

__device__ __forceinline__ v4i mfma_i8(long a, long b) {
    v4i z = {0, 0, 0, 0};
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, z, 0, 0, 0);
}

// B operand (8 signed int8 weights) of an IQ2_XXS record from the LDS tables.
__device__ __forceinline__ long iq2_b_operand(uint32_t rec, const uint32_t* __restrict__ lds_tab) {
    uint32_t lo = lds_tab[rec & 0xFFFu];
    uint32_t hi = lds_tab[4096u + ((rec >> 3) & 0xFFFu)];
    return (long)(((uint64_t)hi << 32) | (uint64_t)lo);
}

// Value of one MFMA output for the (hi, lo) digit rows: exact in int32
// (|256 D_hi + D_lo| <= 256*32*127*127 + ... < 2^31), then one rounding.
__device__ __forceinline__ float digits_combine(int d_hi, int d_lo) {
    return (float)(d_hi * 256 + d_lo);
}

// Cooperative copy of the 32 KiB IQ2_XXS sign/grid tables into LDS.
__device__ __forceinline__ void load_iq2_tables(uint32_t* lds, const uint32_t* __restrict__ g) {
    const uint4* src = reinterpret_cast<const uint4*>(g);
    uint4* dst = reinterpret_cast<uint4*>(lds);
    for (int i = threadIdx.x; i < kIq2TableWords / 4; i += blockDim.x) dst[i] = src[i];
}

// Wave-wide sum (all 64 lanes receive the result).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
    return v;
}

// Quantise one 32-element block held one element per lane of a 32-lane half
// wave: returns this lane's digits and the block scale (same in all 32 lanes).
// Blocks whose max |x| is non-finite get a NaN scale (the block then poisons
// every output that reads it); blocks below 2^-100 are treated as zero.
__device__ __forceinline__ float quantize_block32(float x, int8_t* hi, int8_t* lo) {
    // NaN counts as Inf so that fmaxf (which drops NaN operands) cannot hide it.
    float a = (x != x) ? __uint_as_float(0x7F800000u) : fabsf(x);
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) a = fmaxf(a, __shfl_xor(a, off, 32));
    float scale, inv;
    if (!(a <= 3.4028235e38f)) {            // Inf or NaN in the block
        scale = __uint_as_float(0x7FC00000u);
        inv = 0.0f;
    } else if (a < 0x1p-100f) {
        scale = 0.0f;
        inv = 0.0f;
    } else {
        scale = a / kDigitMax;
        inv = kDigitMax / a;
    }
    float qf = rintf(x * inv);
    qf = fminf(fmaxf(qf, -kDigitMax), kDigitMax);
    int q = (inv == 0.0f) ? 0 : (int)qf;
    int h = (q + 128) >> 8;
    *hi = (int8_t)h;
    *lo = (int8_t)(q - h * 256);
    return scale;
}

}  // namespace mmhip
