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

// IQ2_XXS (dequant.zig:316-369): one thread per 8-weight group.
__global__ void dequant_iq2_kernel(const uint8_t* __restrict__ raw, uint64_t n, float* __restrict__ out) {
    uint64_t grp = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint64_t base = grp * 8;
    if (base >= n) return;
    uint64_t sb = base >> 8;
    uint32_t ib = (uint32_t)((base >> 5) & 7);
    uint32_t l = (uint32_t)((base >> 3) & 3);
    const uint8_t* blk = raw + sb * 66;
    float d = f16_bits_to_f32(ld16(blk));
    uint32_t a0 = ld32u(blk + 2 + 8 * ib);
    uint32_t a1 = ld32u(blk + 2 + 8 * ib + 4);
    float db = d * (0.5f + (float)(a1 >> 28)) * 0.25f;
    uint64_t gv = c_iq2_grid[(a0 >> (8 * l)) & 0xFFu];
    uint32_t code = (a1 >> (7 * l)) & 0x7Fu;
    uint32_t s = code | ((uint32_t)(__popc(code) & 1) << 7);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        if (base + j < n) {
            float mag = (float)((gv >> (8 * j)) & 0xFFu);
            float sign = ((s >> j) & 1u) ? -1.0f : 1.0f;
            out[base + j] = db * mag * sign;
        }
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
    const uint32_t nunit = cols_pad / 256;
    const uint64_t unit = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const uint32_t rows = n_rows ? min(*n_rows, n_max) : n_max;
    if (unit >= (uint64_t)rows * nunit) return;  // whole wave exits together
    quantize_unit_wave<SILU>(src, src_stride, u_off, unit / nunit, (uint32_t)(unit % nunit), cols, hi, lo, sc, q_stride,
                             s_stride);
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
            dequant_q8_0_kernel<<<(unsigned)((n + bs - 1) / bs), bs, 0, s>>>((const uint8_t*)raw, n, out);
            break;
        case kTypeIq2: {
            uint64_t groups = (n + 7) / 8;
            dequant_iq2_kernel<<<(unsigned)((groups + bs - 1) / bs), bs, 0, s>>>((const uint8_t*)raw, n, out);
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
