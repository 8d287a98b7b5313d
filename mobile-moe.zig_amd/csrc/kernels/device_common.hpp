// Device-side building blocks shared by the gfx950 kernels.
//
// Tile layouts (built once at upload by codec.hip; same bytes per block as
// GGUF, only reordered):
//
//   A "row tile" is 16 consecutive output rows. For each row tile the kernels
//   read one 1 KiB record unit per 256 (IQ2_XXS) or 64 (Q8_0) input columns:
//   64 lanes x 16 B, one coalesced 128-bit load per lane. Lane l serves output
//   row n = l % 16 and column group g = l / 16 (8 consecutive columns of each
//   32-column block), which is the B-operand layout of
//   v_mfma_i32_16x16x32_i8 (B[k][n] with k = 8g..8g+7 in lane 16g+n).
//
//   IQ2_XXS unit (one 256-column superblock of 16 rows, 1056 B = 16 x 66 B):
//     recs: lane l holds 4 dwords; dword k covers sub-blocks 2k and 2k+1:
//       bits  0.. 1  two bits of a sub-block scale ls (below)
//       bits  2..16  record of sub-block 2k:   b012 | P<<3 | idx<<4 | hi3<<12
//       bits 17..31  record of sub-block 2k+1 (same fields)
//     where idx = grid index of group g, code = its 7-bit sign code,
//     b012 = code bits 0..2, hi3 = code bits 4..6, P = parity(code bits 0..3).
//     Dwords 0,1 carry ls of sub-block g (bits 0..1, 2..3); dwords 2,3 carry
//     ls of sub-block 4+g. 15 information bits per record + 8 ls bits per lane
//     = the raw format's 64 bits per sub-block-row exactly.
//     d: 16 x f16, one per row.
//   Signed int8 weights come from two 16 KiB LDS tables addressed straight
//   from the dword:  LO[(window b012|P|idx)] = columns 0..3 (signs b0..b3,
//   b3 = P ^ parity(b012)); HI[(window P|idx|hi3)] = columns 4..7 (signs hi3,
//   bit 7 = P ^ parity(hi3), i.e. the ksigns parity bit). Byte addresses:
//   rec 2k:   LO  d & 0x3FFC          HI  (d >> 3) & 0x3FFC
//   rec 2k+1: LO  (d >> 15) & 0x3FFC  HI  (d >> 18) & 0x3FFC
//
//   Q8_0 unit (two 32-column blocks of 16 rows, 1088 B = 32 x 34 B):
//     recs: lane l holds qs[8g..8g+7] of block 2u then of block 2u+1.
//     d:    16 x (f16 d(2u), f16 d(2u+1)).
//
// Activations are quantised per 32-column block to 16-bit fixed point split
// in two int8 digits (x ~= s * (256 * hi + lo)), so one int8 MFMA over a
// 32-column block yields exact integer partial sums for both digits.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

namespace mmhip {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr int kTileRows = 16;
constexpr int kIq2UnitCols = 256;
constexpr int kQ8UnitCols = 64;
constexpr float kDigitMax = 32512.0f;  // 127 * 256: hi digit stays in [-127, 127]
constexpr int kIq2TableWords = 8192;   // LO[4096] then HI[4096], u32 each
// LDS A layout (decode): per 256-column group, lane (m = 0|1, g) owns a
// 64-byte run holding the 8 A operands (8 x 8 digits) of the group's 8
// blocks for A row m (hi/lo digits) and column group g; runs are 80 B apart so
// the 8 lanes' 128-bit reads hit disjoint LDS banks.
constexpr int kARun = 80;
constexpr int kAGroupBytes = 8 * kARun;  // 640 B per 256 columns

// IEEE binary16 bits -> binary32, bit-exact (dequant.zig:19-47 semantics:
// subnormals normalised, Inf/NaN payload kept), independent of the device's
// f16 denormal mode: subnormals are m * 2^-24, computed exactly in f32.
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    uint32_t s = (h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    if (e == 0) return __uint_as_float(s | __float_as_uint((float)m * 0x1p-24f));
    uint32_t bits = (e == 31u) ? (s | 0x7F800000u | (m << 13)) : (s | ((e + 112u) << 23) | (m << 13));
    return __uint_as_float(bits);
}

// Hardware conversion for scales that only feed products: exact for every
// finite value (f16 denormals are enabled for these kernels); NaNs may come
// out quieted, which cannot change a product that is NaN anyway.
__device__ __forceinline__ float f16_scale(uint32_t h) {
    return __half2float(__ushort_as_half((unsigned short)h));
}

__device__ __forceinline__ v4i mfma_i8(long a, long b) {
    v4i z = {0, 0, 0, 0};
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, z, 0, 0, 0);
}

// IQ2_XXS B operands of the two records in one tile dword.
__device__ __forceinline__ long iq2_bop_lo(uint32_t d, const uint32_t* __restrict__ tab) {
    const uint32_t lo = *reinterpret_cast<const uint32_t*>(reinterpret_cast<const char*>(tab) + (d & 0x3FFCu));
    const uint32_t hi = *reinterpret_cast<const uint32_t*>(reinterpret_cast<const char*>(tab) + 16384u +
                                                            ((d >> 3) & 0x3FFCu));
    return (long)(((uint64_t)hi << 32) | (uint64_t)lo);
}
__device__ __forceinline__ long iq2_bop_hi(uint32_t d, const uint32_t* __restrict__ tab) {
    const uint32_t lo = *reinterpret_cast<const uint32_t*>(reinterpret_cast<const char*>(tab) + ((d >> 15) & 0x3FFCu));
    const uint32_t hi = *reinterpret_cast<const uint32_t*>(reinterpret_cast<const char*>(tab) + 16384u +
                                                            ((d >> 18) & 0x3FFCu));
    return (long)(((uint64_t)hi << 32) | (uint64_t)lo);
}

// ls of sub-block g (from dwords 0,1) and 4+g (dwords 2,3) of this lane.
__device__ __forceinline__ uint32_t iq2_ls_a(const uint4& r) { return (r.x & 3u) | ((r.y & 3u) << 2); }
__device__ __forceinline__ uint32_t iq2_ls_b(const uint4& r) { return (r.z & 3u) | ((r.w & 3u) << 2); }

// All eight 4-bit ls values of the lane's row (nibble s = sub-block s),
// gathered from the row's four lanes.
__device__ __forceinline__ uint32_t iq2_ls_all(const uint4& r, uint32_t g) {
    uint32_t mine = (iq2_ls_a(r) << (4 * g)) | (iq2_ls_b(r) << (16 + 4 * g));
    mine |= __shfl_xor(mine, 16, kWave);
    mine |= __shfl_xor(mine, 32, kWave);
    return mine;
}

// Exact integer value of one MFMA output for the (hi, lo) digit rows:
// |256 D_hi + D_lo| <= 256*32*127*127 + 32*127*128 < 2^31.
__device__ __forceinline__ int digits_combine(int d_hi, int d_lo) { return d_hi * 256 + d_lo; }

// Row r (16 lanes) of the result holds v_r's lanes 0..15: four values that
// live in lanes 0..15 of four VGPRs end up one per 16-lane row.
__device__ __forceinline__ int gather_rows4(int v0, int v1, int v2, int v3) {
    auto p = __builtin_amdgcn_permlane16_swap((uint32_t)v0, (uint32_t)v1, false, false);  // [v0 r0, v1 r0, v0 r2, v1 r2]
    auto q = __builtin_amdgcn_permlane16_swap((uint32_t)v2, (uint32_t)v3, false, false);  // [v2 r0, v3 r0, v2 r2, v3 r2]
    auto r = __builtin_amdgcn_permlane32_swap(p[0], q[0], false, false);                  // [v0 r0, v1 r0, v2 r0, v3 r0]
    return (int)r[0];
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
    if (!(a <= 3.4028235e38f)) {
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

// Quantise x[0..cols) into the LDS A layout (kAGroupBytes per 256 columns)
// plus block scales xs[nblk]; blocks cover [0, nblk * 32), zero-padded. All
// threads of the block take part; the caller synchronises afterwards.
__device__ __forceinline__ void quantize_to_lds(const float* __restrict__ x, uint32_t cols, uint32_t nblk,
                                                int8_t* aq, float* xs) {
    constexpr int kBatch = 8;  // blocks per 32-lane group whose loads are in flight together
    const uint32_t groups = blockDim.x >> 5;
    const uint32_t j = threadIdx.x & 31;
    const uint32_t g = j >> 3, jj = j & 7;
    for (uint32_t b0 = threadIdx.x >> 5; b0 < nblk; b0 += groups * kBatch) {
        float v[kBatch];
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
            const uint32_t c = (b0 + i * groups) * 32 + j;
            v[i] = (b0 + i * groups < nblk && c < cols) ? x[c] : 0.0f;
        }
#pragma unroll
        for (int i = 0; i < kBatch; ++i) {
            const uint32_t b = b0 + i * groups;
            if (b >= nblk) break;
            int8_t h, l;
            const float s = quantize_block32(v[i], &h, &l);
            int8_t* run = aq + (b >> 3) * kAGroupBytes + g * kARun + (b & 7) * 8 + jj;
            run[0] = h;
            run[4 * kARun] = l;
            if (j == 0) xs[b] = s;
        }
    }
}

// The 8 A operands (blocks 8G..8G+7 of the LDS chunk) of a lane with
// n = m < 2: four 128-bit reads of its 64-byte run.
__device__ __forceinline__ void lds_a_group(long (&areg)[8], const int8_t* a_run, uint32_t group) {
    const uint4* p = reinterpret_cast<const uint4*>(a_run + group * kAGroupBytes);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint4 q = p[i];
        areg[2 * i] = (long)(((uint64_t)q.y << 32) | q.x);
        areg[2 * i + 1] = (long)(((uint64_t)q.w << 32) | q.z);
    }
}

}  // namespace mmhip
