// Host-side launch API of the gfx950 kernels (implemented in the .hip files
// next to this header). All launches are asynchronous on the given stream and
// return the hipError_t of the launch.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mmhip {

enum TileFormat : uint32_t { kFmtQ8 = 0, kFmtIq2 = 1 };

constexpr int kIq2TableWordsHost = 8192;  // u32 words of the IQ2_XXS LDS tables

// Geometry of a stacked weight in the tile layout (device_common.hpp).
struct TileGeom {
    uint32_t fmt;
    uint64_t rows, cols, count;
    uint64_t tiles;        // ceil(rows / 16)
    uint64_t units;        // record units per row tile
    uint64_t unit_cols;    // 256 (IQ2_XXS) or 64 (Q8_0)
    uint64_t cols_pad;     // units * unit_cols
    uint64_t rec_stride;   // uint4 records per matrix = tiles * units * 64
    uint64_t d_row;        // u16 scales per row, padded: roundup(units * (1 | 2), 8)
    uint64_t d_stride;     // u16 scales per matrix = tiles * 16 * d_row
};

// Quantised activations: 16-bit block fixed point as two int8 digit planes.
struct QuantAct {
    int8_t* hi;
    int8_t* lo;
    float* scale;
    uint64_t stride;       // elements between vectors in hi/lo (>= cols_pad)
    uint64_t scale_stride; // scales between vectors (= stride / 32)
};

struct GemvArgs {
    const uint4* recs;
    const uint16_t* dvals;
    uint64_t rec_stride, d_stride;
    uint32_t d_row;
    const float* x;                 // f32 activations, quantised inside the kernel
    uint64_t x_stride;              // floats between problems' vectors; 0 = shared
    float* y;
    uint64_t y_stride;
    const uint32_t* tables;         // IQ2_XXS LDS tables (32 KiB)
    uint64_t first_mat;
    uint32_t n_probs, tiles, units, rows, cols;
    uint32_t tiles_per_wg;          // set by launch_gemv_q
};

// Raw GGUF bytes -> f32, bit-exact (dequant.zig:316-390, 632-659).
hipError_t launch_dequant(const void* raw, uint32_t ggml_type, uint64_t n, float* out, hipStream_t s);

// Raw GGUF bytes -> tile layout.
hipError_t launch_repack(const void* raw, const TileGeom& g, uint4* recs, uint16_t* dvals, hipStream_t s);

// x [n_vec][cols] (row stride x_stride floats) -> digits + scales; columns in
// [cols, cols_pad) are written as zero.
hipError_t launch_quantize(const float* x, uint64_t x_stride, uint32_t n_vec, uint32_t cols,
                           uint32_t cols_pad, const QuantAct& q, hipStream_t s);

// Quantised-weight GEMV over n_probs matrices in one launch (activations are
// quantised inside the kernel).
hipError_t launch_gemv_q(const GemvArgs& a, uint32_t fmt, int num_cu, hipStream_t s);

// Plain f32 / f16 weight GEMV (router, matVecMulUnified's f32 branch):
// y_i = W_{first+i} . x_i for i < n_mats.
hipError_t launch_gemv_float(const void* w, uint32_t ggml_type, uint64_t mat_stride,
                             const float* x, uint64_t x_stride, float* y, uint64_t y_stride,
                             uint32_t n_mats, uint32_t rows, uint32_t cols, hipStream_t s);

// Batched QMM: Y = X . W^T for `batch` quantised activation rows.
// out_layout 0: y[b * y_ld + r]; 1: y[r * y_ld + b].
hipError_t launch_qmm(const uint4* recs, const uint16_t* dvals, const TileGeom& g, uint64_t mat,
                      const QuantAct& xq, uint32_t batch, float* y, uint64_t y_ld, int out_layout,
                      const uint32_t* tables, hipStream_t s);

// Builds the two IQ2_XXS LDS tables on the host (8192 u32).
void build_iq2_tables(uint32_t* out8192);

}  // namespace mmhip
