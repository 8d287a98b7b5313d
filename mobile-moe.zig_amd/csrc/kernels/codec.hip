// Block codecs on gfx950: bit-exact dequantisation of raw GGUF blocks, the
// one-time repack into the tile layout, and activation quantisation.
#include "device_common.hpp"
#include "kernels.hpp"

namespace mmhip {

namespace {

constexpr uint32_t kTypeF32 = 0, kTypeF16 = 1, kTypeQ8_0 = 8, kTypeIq2 = 16;

// Raw GGUF bytes are only 2-byte aligned (34 / 66-byte blocks): read u16s.
__device__ __forceinline__ uint32_t ld16(const uint8_t* p) {
    return (uint32_t)*reinterpret_cast<const uint16_t*>(p);
}
__device__ __forceinline__ uint32_t ld32u(const uint8_t* p) {
    return ld16(p) | (ld16(p + 2) << 16);
}

// Q8_0 (dequant.zig:379-390): one thread per output element.
__global__ void dequant_q8_0_kernel(const uint8_t* __restrict__ raw, uint64_t n, float* __restrict__ out) {
    uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint8_t* blk = raw + (i >> 5) * 34;
    float d = f16_bits_to_f32(ld16(blk));
    out[i] = d * (float)(int8_t)blk[2 + (i & 31)];
}

// IQ2_XXS (dequant.zig:316-369): one thread per half of an 8-weight group,
// so that consecutive lanes write consecutive 16 bytes: one non-temporal
// float4 store per thread (whole cache lines per instruction) when out is
// 16-byte aligned.
__global__ void dequant_iq2_kernel(const uint8_t* __restrict__ raw, uint64_t n, bool vec, float* __restrict__ out) {
    const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t base = t * 4;
    if (base >= n) return;
    const uint32_t h = (uint32_t)(t & 1);
    const uint64_t sb = base >> 8;
    const uint32_t ib = (uint32_t)((base >> 5) & 7);
    const uint32_t l = (uint32_t)((base >> 3) & 3);
    const uint8_t* blk = raw + sb * 66;
    const float d = f16_bits_to_f32(ld16(blk));
    const uint32_t a0 = ld32u(blk + 2 + 8 * ib);
    const uint32_t a1 = ld32u(blk + 2 + 8 * ib + 4);
    const float db = d * (0.5f + (float)(a1 >> 28)) * 0.25f;
    const uint64_t gv = c_iq2_grid[(a0 >> (8 * l)) & 0xFFu];
    const uint32_t code = (a1 >> (7 * l)) & 0x7Fu;
    const uint32_t sg = code | ((uint32_t)(__popc(code) & 1) << 7);
    float v[4];
#pragma unroll
    for (uint32_t e = 0; e < 4; ++e) {
        const uint32_t j = 4 * h + e;
        const float mag = (float)((gv >> (8 * j)) & 0xFFu);
        const float sign = ((sg >> j) & 1u) ? -1.0f : 1.0f;
        v[e] = db * mag * sign;
    }
    if (vec && base + 4 <= n) {
        typedef float v4f_ __attribute__((ext_vector_type(4)));
        __builtin_nontemporal_store(v4f_{v[0], v[1], v[2], v[3]}, reinterpret_cast<v4f_*>(out + base));
    } else {
#pragma unroll
        for (uint32_t e = 0; e < 4; ++e)
            if (base + e < n) out[base + e] = v[e];
    }
}

__global__ void dequant_f16_kernel(const uint16_t* __restrict__ raw, uint64_t n, float* __restrict__ out) {
    uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = f16_bits_to_f32(raw[i]);
}

// Raw IQ2_XXS -> tile records (layout in device_common.hpp). One thread per
// (matrix, row tile, superblock column, lane).
__global__ void repack_iq2_kernel(const uint8_t* __restrict__ raw, uint64_t rows, uint64_t nsb,
                                  uint64_t tiles, uint64_t total, uint64_t d_row, uint4* __restrict__ recs,
                                  uint16_t* __restrict__ dvals) {
    uint64_t gid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= total) return;
    uint32_t lane = (uint32_t)(gid & 63);
    uint64_t unit = gid >> 6;
    uint64_t j = unit % nsb;
    uint64_t t = (unit / nsb) % tiles;
    uint64_t mat = unit / (nsb * tiles);
    uint32_t n = lane & 15, g = lane >> 4;
    uint64_t row = t * 16 + n;
    uint32_t w[4] = {0, 0, 0, 0};
    uint32_t dbits = 0;
    if (row < rows) {
        const uint8_t* sb = raw + ((mat * rows + row) * nsb + j) * 66;
        dbits = ld16(sb);
        uint32_t la = 0, lb = 0;
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            uint32_t a0 = ld32u(sb + 2 + 8 * s);
            uint32_t a1 = ld32u(sb + 2 + 8 * s + 4);
            uint32_t idx = (a0 >> (8 * g)) & 0xFFu;
            uint32_t code = (a1 >> (7 * g)) & 0x7Fu;
            if ((uint32_t)s == g) la = a1 >> 28;
            if ((uint32_t)s == 4 + g) lb = a1 >> 28;
            const uint32_t window = (code & 7u) | ((uint32_t)(__popc(code & 15u) & 1) << 3) | (idx << 4);
            const uint32_t hi3 = (code >> 4) & 7u;
            w[s >> 1] |= (s & 1) ? ((window << 18) | hi3) : ((window << 3) | (hi3 << 15));
        }
        // ls of sub-block g in dwords 0,1 and of sub-block 4+g in dwords 2,3.
        w[0] |= (la & 3u) << 30;
        w[1] |= (la >> 2) << 30;
        w[2] |= (lb & 3u) << 30;
        w[3] |= (lb >> 2) << 30;
    }
    recs[gid] = make_uint4(w[0], w[1], w[2], w[3]);
    if (g == 0) dvals[((mat * tiles + t) * 16 + n) * d_row + j] = (uint16_t)dbits;
}

// Raw Q8_0 -> tile records: a unit is two 32-column blocks of 16 rows.
__global__ void repack_q8_kernel(const uint8_t* __restrict__ raw, uint64_t rows, uint64_t nb,
                                 uint64_t nu, uint64_t tiles, uint64_t total, uint64_t d_row,
                                 uint4* __restrict__ recs, uint16_t* __restrict__ dvals) {
    uint64_t gid = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (gid >= total) return;
    uint32_t lane = (uint32_t)(gid & 63);
    uint64_t unit = gid >> 6;
    uint64_t u = unit % nu;
    uint64_t t = (unit / nu) % tiles;
    uint64_t mat = unit / (nu * tiles);
    uint32_t n = lane & 15, g = lane >> 4;
    uint64_t row = t * 16 + n;
    uint32_t w[4] = {0, 0, 0, 0};
    uint32_t dbits[2] = {0, 0};
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        uint64_t blk = 2 * u + b;
        if (row < rows && blk < nb) {
            const uint8_t* src = raw + ((mat * rows + row) * nb + blk) * 34;
            dbits[b] = ld16(src);
            const uint8_t* q = src + 2 + 8 * g;
            w[2 * b] = ld32u(q);
            w[2 * b + 1] = ld32u(q + 4);
        }
    }
    recs[gid] = make_uint4(w[0], w[1], w[2], w[3]);
    if (g == 0) {
        uint16_t* dr = dvals + ((mat * tiles + t) * 16 + n) * d_row + 2 * u;
        dr[0] = (uint16_t)dbits[0];
        dr[1] = (uint16_t)dbits[1];
    }
}

// One 32-lane group per 32-column block.
__global__ void quantize_kernel(const float* __restrict__ x, uint64_t x_stride, uint32_t n_vec,
                                uint32_t cols, uint32_t cols_pad, int8_t* __restrict__ hi,
                                int8_t* __restrict__ lo, float* __restrict__ sc, uint64_t q_stride,
                                uint64_t s_stride) {
    uint32_t nblk = cols_pad / 32;
    uint64_t blk = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 5;
    uint32_t j = threadIdx.x & 31;
    if (blk >= (uint64_t)n_vec * nblk) return;  // whole 32-lane group exits together
    uint64_t v = blk / nblk;
    uint32_t b = (uint32_t)(blk % nblk);
    uint32_t col = b * 32 + j;
    float xv = col < cols ? x[v * x_stride + col] : 0.0f;
    int8_t h, l;
    float s = quantize_block32(xv, &h, &l);
    hi[v * q_stride + col] = h;
    lo[v * q_stride + col] = l;
    if (j == 0) sc[v * s_stride + b] = s;
}

// silu(g) * u per row, then as quantize_kernel; rows r >= *n_rows are skipped.
__global__ void quantize_silu_kernel(const float* __restrict__ src, uint64_t src_stride, uint64_t u_off,
                                     const uint32_t* __restrict__ n_rows, uint32_t n_max, uint32_t cols,
                                     uint32_t cols_pad, int8_t* __restrict__ hi, int8_t* __restrict__ lo,
                                     float* __restrict__ sc, uint64_t q_stride, uint64_t s_stride) {
    const uint32_t nblk = cols_pad / 32;
    const uint64_t blk = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 5;
    const uint32_t j = threadIdx.x & 31;
    const uint32_t rows = n_rows ? min(*n_rows, n_max) : n_max;
    if (blk >= (uint64_t)rows * nblk) return;  // whole 32-lane group exits together
    const uint64_t v = blk / nblk;
    const uint32_t b = (uint32_t)(blk % nblk);
    const uint32_t col = b * 32 + j;
    float xv = 0.0f;
    if (col < cols) {
        const float* g = src + v * src_stride;
        xv = silu(g[col]) * g[u_off + col];
    }
    int8_t h, l;
    const float s = quantize_block32(xv, &h, &l);
    hi[v * q_stride + col] = h;
    lo[v * q_stride + col] = l;
    if (j == 0) sc[v * s_stride + b] = s;
}

// Wide variants: one wave per 256-column unit (4 columns per lane), one
// scale per unit stored into the unit's eight block slots. src_stride /
// u_off as quantize_silu_kernel; silu == 0: plain quantisation of x.
template <bool SILU>
__global__ __launch_bounds__(256) void quantize_wide_kernel(const float* __restrict__ src, uint64_t src_stride,
                                                             uint64_t u_off, const uint32_t* __restrict__ n_rows,
                                                             uint32_t n_max, uint32_t cols, uint32_t cols_pad,
                                                             int8_t* __restrict__ hi, int8_t* __restrict__ lo,
                                                             float* __restrict__ sc, uint64_t q_stride,
                                                             uint64_t s_stride) {
    // All arguments in one batch of scalar loads (the early exit below
    // otherwise waited for its own first: one more round trip).
    asm volatile("" ::"s"(src), "s"(src_stride), "s"(u_off), "s"(n_rows), "s"(n_max), "s"(cols), "s"(cols_pad),
                 "s"(hi), "s"(lo), "s"(sc), "s"(q_stride), "s"(s_stride));
    const uint32_t nunit = cols_pad / 256;
    const uint64_t unit = ((uint64_t)blockIdx.x * 256 + threadIdx.x) >> 6;  // 256 threads (launch_quantize*)
    const uint32_t rows = n_rows ? min(*n_rows, n_max) : n_max;
    if (unit >= (uint64_t)rows * nunit) return;  // whole wave exits together
    quantize_unit_wave<SILU>(src, src_stride, u_off, unit / nunit, (uint32_t)(unit % nunit), cols, hi, lo, sc, q_stride,
                             s_stride);
}

// ---- Q8_0 codec over rows (quantizeQ8_0, dequant.zig:98-130; the Q8_0
// branches of KVCache.put / getKVCompressed / getKPe, kv_cache.zig:225-349) ----
//
// Row r of row_len values maps to ceil(row_len / 32) blocks of 34 bytes at
// r * ceil(row_len / 32) * 34; a row's last block is padded with zeros. One
// wave covers 8 consecutive blocks of the flattened (row, block) order: lane
// (k, j) holds values 4j..4j+3 of block k, so the wave reads 1 KiB of
// activations (contiguous within a row) and writes 272 bytes, assembled in
// LDS and stored as dwords (a wave's output starts at a multiple of 272).

// f32ToF16 (dequant.zig:50-95) as the quantiser stores a block scale: round
// to nearest even on the normal range, 0 for f32 subnormals and below 2^-25,
// Inf / NaN kept. On the f16 subnormal range, [2^-25, 2^-14), the reference
// shifts the significand by 1 - e16, which spills out of the 10-bit field: a
// trap in safe builds for [2^-21, 2^-14), a corrupted code for [2^-25, 2^-21)
// (2^-22 -> 0x8000). This takes the branch's evident intent on the whole
// range, a shift by 14 - e16: the subnormal value truncated toward zero.
__device__ __forceinline__ uint32_t f32_to_f16_scale(float v) {
    const uint32_t bits = __float_as_uint(v);
    const uint32_t er = (bits >> 23) & 0xFFu, mant = bits & 0x7FFFFFu;
    uint32_t e = 0, m = 0;
    if (er == 0xFFu) {
        e = 0x1Fu;
        m = mant >> 13;
        if (mant != 0 && m == 0) m = 1;
    } else if (er != 0) {
        const int e16 = (int)er - 112;
        if (e16 >= 31) {
            e = 0x1Fu;
        } else if (e16 <= 0) {
            if (e16 >= -10) m = (mant | 0x800000u) >> (uint32_t)(14 - e16);
        } else {
            e = (uint32_t)e16;
            m = mant >> 13;
            const uint32_t rb = mant & 0x1FFFu;
            if (rb > 0x1000u || (rb == 0x1000u && (m & 1u))) {
                ++m;
                if (m == 0x400u) {
                    m = 0;
                    ++e;
                }
            }
        }
    }
    return ((bits >> 31) << 15) | (e << 10) | m;
}

// Tiles of 256 consecutive blocks (8,704 bytes: 68 whole 128-byte lines of
// the block array) per 512-thread workgroup: lane (k, j) holds values
// 4j..4j+3 of blocks k + 64u, u < 4, all four loads issued before any use
// (~128 KiB in flight per CU at four workgroups, which HBM latency needs);
// workgroups loop over tiles. The f32 input is read and the blocks written
// non-temporally (each byte is touched once).
constexpr int kQ8Threads = 512;
constexpr uint32_t kQ8Groups = kQ8Threads / 8;  // blocks per pass of the workgroup
constexpr uint32_t kQ8Per = 4;                  // passes per tile
constexpr uint32_t kQ8TileBlocks = kQ8Groups * kQ8Per;
constexpr uint32_t kQ8TileWords = kQ8TileBlocks * 34 / 4;
constexpr uint64_t kQ8Grid = 256 * 4;  // workgroups: 4 per CU of MI355X

// Row and block-in-row of block b0 + k, from (row0, blk0) = b0 split once per
// tile: (blk0 + k) / bpr by a float reciprocal, corrected by one step (the
// quotient is below 2^16, so the estimate is off by at most one).
struct RowBlock {
    uint64_t row;
    uint32_t blk;
};
__device__ __forceinline__ RowBlock row_block(uint64_t row0, uint32_t blk0, uint32_t k, uint32_t bpr, float inv_bpr) {
    // t < bpr + 2^10 < 2^28 (row_len < 2^32), so q * bpr <= t + bpr fits in
    // 32 bits. 24-bit multiplies (full rate) need both factors below 2^24,
    // which holds for q always and for bpr on rows of fewer than 2^29
    // values; longer rows take the 32-bit multiplies (the branch is uniform).
    const uint32_t t = blk0 + k;
    uint32_t q = (uint32_t)((float)t * inv_bpr);
    if (bpr < (1u << 24)) {
        if (__umul24(q, bpr) > t) --q;
        if (__umul24(q + 1, bpr) <= t) ++q;
        return RowBlock{row0 + q, t - __umul24(q, bpr)};
    }
    if (q * bpr > t) --q;
    if ((q + 1) * bpr <= t) ++q;
    return RowBlock{row0 + q, t - q * bpr};
}

__global__ __launch_bounds__(kQ8Threads) void quantize_q8_0_rows_kernel(const float* __restrict__ x,
                                                                        uint64_t x_stride, uint64_t n_rows,
                                                                        uint32_t row_len, bool vec,
                                                                        uint8_t* __restrict__ out) {
    __shared__ __align__(16) uint32_t stage[kQ8TileWords];
    uint8_t* const st = reinterpret_cast<uint8_t*>(stage);
    const uint32_t k = threadIdx.x >> 3, j = threadIdx.x & 7;
    const uint32_t bpr = (row_len + 31) / 32;
    const float inv_bpr = 1.0f / (float)bpr;
    const uint64_t nblk = n_rows * bpr;
    const uint64_t n_tiles = (nblk + kQ8TileBlocks - 1) / kQ8TileBlocks;
    for (uint64_t tile = blockIdx.x; tile < n_tiles; tile += gridDim.x) {
        const uint64_t b0 = tile * kQ8TileBlocks;
        const uint64_t row0 = b0 / bpr;
        const uint32_t blk0 = (uint32_t)(b0 % bpr);
        float v[kQ8Per][4];
        uint32_t n_live[kQ8Per];
#pragma unroll
        for (uint32_t u = 0; u < kQ8Per; ++u) {
            const uint32_t kk = k + kQ8Groups * u;
            const RowBlock rb = row_block(row0, blk0, kk, bpr, inv_bpr);
            const uint32_t c0 = rb.blk * 32 + 4 * j;
            // Values past the row (or past the last block) count as absent.
            n_live[u] = b0 + kk < nblk ? (c0 < row_len ? min(row_len - c0, 4u) : 0u) : 0u;
            const float* src = x + rb.row * x_stride + c0;
#pragma unroll
            for (int e = 0; e < 4; ++e) v[u][e] = 0.0f;
            if (vec && n_live[u] == 4) {
                typedef float v4f_ __attribute__((ext_vector_type(4)));
                const v4f_ qv = __builtin_nontemporal_load(reinterpret_cast<const v4f_*>(src));
                const float4 q = make_float4(qv[0], qv[1], qv[2], qv[3]);
                v[u][0] = q.x;
                v[u][1] = q.y;
                v[u][2] = q.z;
                v[u][3] = q.w;
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if ((uint32_t)e < n_live[u]) v[u][e] = src[e];
            }
        }
#pragma unroll
        for (uint32_t u = 0; u < kQ8Per; ++u) {
            // The block's largest |x| (a NaN never compares greater).
            float m = 0.0f;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float av = fabsf(v[u][e]);
                m = ((uint32_t)e < n_live[u] && av > m) ? av : m;
            }
            m = max8_lanes(m);
            const float d = m > 0.0f ? m / 127.0f : 0.0f;
            // x / d rounded half away from zero (@round of the f32 quotient).
            // z = x * rcp(d) is within |x/d| * (2^-23 + 2^-24) <= 2.3e-5 of
            // the exact quotient (rcp: 1 ulp; |x/d| <= 127.00002), and the
            // correctly rounded quotient is within 2^-17 of it; where z is
            // more than 1e-4 from every half-integer both round to the same
            // integer. Lanes with a value closer, with |z| > 127.25 (a
            // subnormal d can push the quotient past 127.5, which the exact
            // path clamps) or with a non-finite z (d = 0, Inf or NaN inputs)
            // redo their block with the IEEE division.
            const float rd = __builtin_amdgcn_rcpf(d);
            uint32_t q4 = 0;
            bool near = false;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                // y = |z| + 0.5 (rounding error <= 2^-18 for |z| < 128): |z| is
                // near a half-integer where y is near an integer.
                const float z = v[u][e] * rd, az = fabsf(z), y = az + 0.5f, r = truncf(y);
                near |= !(az <= 127.25f) || !(fabsf((y - r) - 0.5f) < 0.5f - 1.0e-4f);
                // Not near: |z| <= 127.25 and away from half-integers, so the
                // rounded value is in [-127, 127]; absent values are 0.
                q4 |= ((uint32_t)(int)copysignf(r, z) & 0xFFu) << (8 * e);
            }
            if (__any(near) && near) {
                q4 = 0;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float r = roundf(v[u][e] / d);
                    const float re = (r == r && d > 0.0f && (uint32_t)e < n_live[u]) ? r : 0.0f;  // NaN input (@intFromFloat traps)
                    const int q = (int)fminf(fmaxf(re, -127.0f), 127.0f);
                    q4 |= (uint32_t)(q & 0xFF) << (8 * e);
                }
            }
            const uint32_t kk = k + kQ8Groups * u;
            if (b0 + kk < nblk) {
                *reinterpret_cast<uint16_t*>(st + kk * 34 + 2 + 4 * j) = (uint16_t)(q4 & 0xFFFFu);
                *reinterpret_cast<uint16_t*>(st + kk * 34 + 4 + 4 * j) = (uint16_t)(q4 >> 16);
                if (j == 0) *reinterpret_cast<uint16_t*>(st + kk * 34) = (uint16_t)f32_to_f16_scale(d);
            }
        }
        lds_barrier();
        const uint32_t bytes = (uint32_t)min<uint64_t>(kQ8TileBlocks, nblk - b0) * 34;
        uint8_t* dst = out + b0 * 34;  // 4-byte aligned: b0 * 34 is a multiple of 8,704
        for (uint32_t i = threadIdx.x; i < bytes / 4; i += kQ8Threads)
            __builtin_nontemporal_store(stage[i], reinterpret_cast<uint32_t*>(dst) + i);
        if ((bytes & 3u) && threadIdx.x == 0)
            *reinterpret_cast<uint16_t*>(dst + bytes - 2) = *reinterpret_cast<const uint16_t*>(st + bytes - 2);
        lds_barrier();  // the tile's LDS is free again
    }
}

// Rows of row_len values back from their blocks: out[r * out_stride + c] =
// f16ToF32(d) * q (dequantizeQ8_0, dequant.zig:379-390; exact in f32). One
// short-lived wave per 8 blocks (lane (k, j): values 4j..4j+3 of block k):
// the output is 4x the input, and many small workgroups keep the stores
// streaming better than a loop over tiles. The float4 stores are
// non-temporal: written through without being kept in the caches, the call
// runs at 7.4 TB/s against 4.3 TB/s with ordinary stores (131,072 x 576).
constexpr int kQ8DqThreads = 256;
__global__ __launch_bounds__(kQ8DqThreads) void dequantize_q8_0_rows_kernel(const uint8_t* __restrict__ blocks,
                                                                            uint64_t n_rows, uint32_t row_len,
                                                                            float inv_bpr, double inv_bpr_d, bool vec,
                                                                            float* __restrict__ out,
                                                                            uint64_t out_stride) {
    const uint32_t k = (threadIdx.x >> 3) & 7, j = threadIdx.x & 7;
    const uint32_t bpr = (row_len + 31) / 32;
    const uint64_t nblk = n_rows * bpr;
    const uint64_t b0 = ((uint64_t)blockIdx.x * (kQ8DqThreads / 64) + (threadIdx.x >> 6)) * 8;
    if (b0 + k >= nblk) return;
    // b0 / bpr from the host's reciprocals (a wave writes only 1 KiB, so an
    // integer division per wave would cost more than its stores): the double
    // estimate is within one of the quotient for b0 < 2^50, then corrected.
    uint64_t row0 = (uint64_t)((double)b0 * inv_bpr_d);
    if (row0 * bpr > b0) --row0;
    else if ((row0 + 1) * bpr <= b0) ++row0;
    const RowBlock rb = row_block(row0, (uint32_t)(b0 - row0 * bpr), k, bpr, inv_bpr);
    const uint8_t* blk = blocks + (b0 + k) * 34;
    const float d = f16_scale(*reinterpret_cast<const uint16_t*>(blk));
    const uint32_t q4 = (uint32_t)*reinterpret_cast<const uint16_t*>(blk + 2 + 4 * j) |
                        ((uint32_t)*reinterpret_cast<const uint16_t*>(blk + 4 + 4 * j) << 16);
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = d * (float)(int8_t)(q4 >> (8 * e));
    const uint32_t c0 = rb.blk * 32 + 4 * j;
    float* dst = out + rb.row * out_stride + c0;
    if (vec && c0 + 4 <= row_len) {
        typedef float v4f_ __attribute__((ext_vector_type(4)));
        __builtin_nontemporal_store(v4f_{v[0], v[1], v[2], v[3]}, reinterpret_cast<v4f_*>(dst));
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (c0 + e < row_len) dst[e] = v[e];
    }
}

}  // namespace

hipError_t launch_dequant(const void* raw, uint32_t type, uint64_t n, float* out, hipStream_t s) {
    if (n == 0) return hipSuccess;
    const int bs = 256;
    switch (type) {
        case kTypeF32:
            return hipMemcpyAsync(out, raw, n * 4, hipMemcpyDeviceToDevice, s);
        case kTypeF16:
            dequant_f16_kernel<<<(unsigned)((n + bs - 1) / bs), bs, 0, s>>>((const uint16_t*)raw, n, out);
            break;
        case kTypeQ8_0:
            // As one row of n values (the KV codec's dequantiser: float4
            // non-temporal stores) where its limits allow.
            if ((reinterpret_cast<uintptr_t>(raw) & 1u) == 0 && n <= 0xFFFFFFFFull)
                return launch_dequantize_q8_0_rows(raw, 1, (uint32_t)n, out, (n + 3) & ~3ull, s);  // one row: the stride is unused
            dequant_q8_0_kernel<<<(unsigned)((n + bs - 1) / bs), bs, 0, s>>>((const uint8_t*)raw, n, out);
            break;
        case kTypeIq2: {
            const uint64_t quads = (n + 3) / 4;
            const bool vec = (reinterpret_cast<uintptr_t>(out) & 15u) == 0;
            dequant_iq2_kernel<<<(unsigned)((quads + bs - 1) / bs), bs, 0, s>>>((const uint8_t*)raw, n, vec, out);
            break;
        }
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_repack(const void* raw, const TileGeom& g, uint4* recs, uint16_t* dvals, hipStream_t s) {
    uint64_t total = g.count * g.tiles * g.units * 64;
    if (total == 0) return hipSuccess;
    const int bs = 256;
    unsigned grid = (unsigned)((total + bs - 1) / bs);
    if (g.fmt == kFmtIq2) {
        repack_iq2_kernel<<<grid, bs, 0, s>>>((const uint8_t*)raw, g.rows, g.units, g.tiles, total, g.d_row, recs,
                                              dvals);
    } else {
        uint64_t nb = (g.cols + 31) / 32;
        repack_q8_kernel<<<grid, bs, 0, s>>>((const uint8_t*)raw, g.rows, nb, g.units, g.tiles, total, g.d_row, recs,
                                             dvals);
    }
    return hipGetLastError();
}

hipError_t launch_quantize(const float* x, uint64_t x_stride, uint32_t n_vec, uint32_t cols,
                           uint32_t cols_pad, const QuantAct& q, hipStream_t s, bool wide) {
    uint64_t threads = (uint64_t)n_vec * cols_pad;
    if (threads == 0) return hipSuccess;
    const int bs = 256;
    if (wide) {
        if (cols_pad % 256) return hipErrorInvalidValue;
        quantize_wide_kernel<false><<<(unsigned)((threads / 4 + bs - 1) / bs), bs, 0, s>>>(
            x, x_stride, 0, nullptr, n_vec, cols, cols_pad, q.hi, q.lo, q.scale, q.stride, q.scale_stride);
        return hipGetLastError();
    }
    quantize_kernel<<<(unsigned)((threads + bs - 1) / bs), bs, 0, s>>>(
        x, x_stride, n_vec, cols, cols_pad, q.hi, q.lo, q.scale, q.stride, q.scale_stride);
    return hipGetLastError();
}

hipError_t launch_quantize_silu(const float* src, uint64_t src_stride, uint64_t u_off, const uint32_t* n_rows,
                                uint32_t n_rows_max, uint32_t cols, uint32_t cols_pad, const QuantAct& q,
                                hipStream_t s, bool wide) {
    const uint64_t threads = (uint64_t)n_rows_max * cols_pad;
    if (threads == 0) return hipSuccess;
    const int bs = 256;
    if (wide) {
        if (cols_pad % 256) return hipErrorInvalidValue;
        quantize_wide_kernel<true><<<(unsigned)((threads / 4 + bs - 1) / bs), bs, 0, s>>>(
            src, src_stride, u_off, n_rows, n_rows_max, cols, cols_pad, q.hi, q.lo, q.scale, q.stride,
            q.scale_stride);
        return hipGetLastError();
    }
    quantize_silu_kernel<<<(unsigned)((threads + bs - 1) / bs), bs, 0, s>>>(
        src, src_stride, u_off, n_rows, n_rows_max, cols, cols_pad, q.hi, q.lo, q.scale, q.stride, q.scale_stride);
    return hipGetLastError();
}

}  // namespace mmhip

namespace mmhip {

hipError_t launch_quantize_q8_0_rows(const float* x, uint64_t x_stride, uint64_t n_rows, uint32_t row_len, void* out,
                                     hipStream_t s) {
    if (n_rows == 0 || row_len == 0) return hipSuccess;
    if (reinterpret_cast<uintptr_t>(out) & 3u) return hipErrorInvalidValue;
    const uint64_t tiles = (n_rows * ((row_len + 31) / 32) + kQ8TileBlocks - 1) / kQ8TileBlocks;
    const bool vec = (reinterpret_cast<uintptr_t>(x) & 15u) == 0 && x_stride % 4 == 0;
    const unsigned grid = (unsigned)(tiles < kQ8Grid ? tiles : kQ8Grid);
    quantize_q8_0_rows_kernel<<<grid, kQ8Threads, 0, s>>>(x, x_stride, n_rows, row_len, vec,
                                                           static_cast<uint8_t*>(out));
    return hipGetLastError();
}

hipError_t launch_dequantize_q8_0_rows(const void* blocks, uint64_t n_rows, uint32_t row_len, float* out,
                                       uint64_t out_stride, hipStream_t s) {
    if (n_rows == 0 || row_len == 0) return hipSuccess;
    if (reinterpret_cast<uintptr_t>(blocks) & 1u) return hipErrorInvalidValue;
    const uint64_t nblk = n_rows * ((row_len + 31) / 32);
    const uint64_t per_wg = (uint64_t)(kQ8DqThreads / 64) * 8;
    const bool vec = (reinterpret_cast<uintptr_t>(out) & 15u) == 0 && out_stride % 4 == 0;
    const uint32_t bpr = (row_len + 31) / 32;
    dequantize_q8_0_rows_kernel<<<(unsigned)((nblk + per_wg - 1) / per_wg), kQ8DqThreads, 0, s>>>(
        static_cast<const uint8_t*>(blocks), n_rows, row_len, 1.0f / (float)bpr, 1.0 / (double)bpr, vec, out,
        out_stride);
    return hipGetLastError();
}

}  // namespace mmhip
