// Host-side launch API of the gfx950 kernels (implemented in the .hip files
// next to this header). All launches are asynchronous on the given stream and
// return the hipError_t of the launch.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mmhip {

enum TileFormat : uint32_t { kFmtQ8 = 0, kFmtIq2 = 1 };

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

// One item of a grouped (expert-sorted) QMM: rows [slot, slot + count) of the
// activation list against matrix `mat`; count <= kQmmTokens.
struct QmmWork {
    uint32_t mat, slot, count, pad;
};
constexpr uint32_t kQmmTokens = 8;  // activation rows per QMM work item

struct RouteArgs {
    const float* scores;        // [n_tokens][n_experts]
    uint32_t n_tokens, n_experts;
    uint32_t k;                 // min(active_expert_limit, 4), >= 1
    int32_t level;              // throttle level 0..3
    float scale;                // getRoutedScalingFactor
    uint32_t shared;            // 1: the layer has a shared expert
    uint32_t shared_merged;     // 1: shared gate/up are matrices 2E, 2E+1 and shared down is matrix E
    unsigned long long* counts; // ExpertStats.counts of the layer [n_experts]
    uint32_t* route_ids;        // [n_tokens][4] or null
    float* route_w;             // [n_tokens][4] or null
    int32_t* assign_slot;       // [n_tokens][4]: slot of (t, i), -1 = none (skipped or i >= k)
    float* assign_w;            // [n_tokens][4]
    int32_t* shared_slot;       // [n_tokens]: slot of the shared expert, -1 = none
    uint32_t* deferred;         // [n_tokens]
    uint32_t* slot_tok;         // [5 n_tokens]: token of each slot
    uint4* gemv_gu;             // n_tokens == 1: {matrix, 0, 2 slot + (0 gate | 1 up), 0}
    uint4* gemv_dn;             //                {matrix, slot, slot, 0}
    uint32_t* n_gemv;           // [2]: active entries of gemv_gu, gemv_dn
    QmmWork* work_gu;           // n_tokens > 1: grouped items (gate col 0, up col inter)
    QmmWork* work_dn;
    uint32_t* n_work;           // [2]: active items of work_gu, work_dn
    uint32_t inter;             // routed expert width (up column offset)
    // Optional, n_tokens > 1: the hidden states' wide quantisation (one
    // scale per 256 columns) for the grouped gate/up, done by extra
    // workgroups of the routing launch (it does not depend on the routing).
    const float* qx = nullptr;  // [n_tokens][qx_stride]; null: no quantisation
    uint64_t qx_stride = 0;
    uint32_t q_cols = 0, q_units = 0;  // columns, 256-column units (cols_pad / 256)
    QuantAct qa{};
};

struct GemvArgs {
    const uint4* recs;
    const uint16_t* dvals;
    uint64_t rec_stride, d_stride;
    uint32_t d_row;
    const float* x;                 // f32 activations, quantised inside the kernel
    uint64_t x_stride;              // floats between problems' vectors; 0 = shared
    uint64_t x2_off;                // silu_mul: floats from a problem's x to its second vector
    uint32_t silu_mul;              // 1: the activation is silu(x) * x2 (expertFFN, inference.zig:1179-1180)
    float* y;
    uint64_t y_stride;
    uint64_t first_mat;
    const uint4* probs;             // device [n_probs] {matrix, x row, y row, 0}, or null: (first_mat + p, p, p)
    const uint32_t* n_active;       // device: problems p >= *n_active do nothing, or null
    uint32_t n_probs, tiles, units, rows, cols;
    uint32_t tiles_per_wg;          // set by launch_gemv_q
    // Decode gate/up (route_decode = 1): the problems come from routing the
    // single token's scores (route.scores) inside the kernel, not from probs /
    // n_active: problem 2s + h is half h (0 gate, 1 up) of the s-th computed
    // assignment (matrix id or E + id, y row 2s + h), then the merged shared
    // expert's gate / up (matrices 2E, 2E+1, y rows 8, 9). Workgroup (0, 0)
    // also writes the routing outputs the later kernels read (route ids and
    // weights, statistics, slots, the down problem list).
    RouteArgs route{};
    uint32_t route_decode = 0;
};


// Arguments of a call with one segment, no problem list and no silu_mul
// (a single matrix, or n_probs matrices and vectors at fixed strides), for
// the decode GEMVs' *_one_kernel entries: the fields the first loads depend
// on arrive as scalar kernel arguments, which the hardware preloads into
// SGPRs (the
// compiler preloads leading scalar arguments, not a struct), so no load
// waits for a kernel-argument round trip; the rest is read from the
// GemvArgs, where nothing needs it before the stores. recs and dvals already
// point at the first matrix; strides are in 16-byte records, f16 scales and
// floats.
struct GemvOneArgs {
    const uint4* recs;
    const uint16_t* dvals;
    const float* x;
    uint32_t rec_stride, d_stride, x_stride;
    uint32_t cols, units, tiles_per_wg, tiles, n_probs, d_row;
    static constexpr uint64_t first_mat = 0, x2_off = 0;
    static constexpr uint32_t silu_mul = 0;
    static constexpr const uint4* probs = nullptr;
    static constexpr const uint32_t* n_active = nullptr;
};

// Raw GGUF bytes -> f32, bit-exact (dequant.zig:316-390, 632-659).
hipError_t launch_dequant(const void* raw, uint32_t ggml_type, uint64_t n, float* out, hipStream_t s);

// Q8_0 codec over rows (quantizeQ8_0, dequant.zig:98-130; KVCache.put /
// getKVCompressed's Q8_0 branches): row r of row_len floats <-> ceil(row_len
// / 32) 34-byte blocks at r * ceil(row_len / 32) * 34. out of the quantiser
// 4-byte aligned, blocks of the dequantiser 2-byte aligned.
hipError_t launch_quantize_q8_0_rows(const float* x, uint64_t x_stride, uint64_t n_rows, uint32_t row_len, void* out,
                                     hipStream_t s);
hipError_t launch_dequantize_q8_0_rows(const void* blocks, uint64_t n_rows, uint32_t row_len, float* out,
                                       uint64_t out_stride, hipStream_t s);

// sampleGreedy (inference.zig:376-386): *out = the first index of the
// largest of n logits (a NaN never wins; a NaN x[0] gives 0). 1 <= n < 2^32;
// scratch holds argmax_scratch_bytes(n) bytes of device memory.
uint64_t argmax_scratch_bytes(uint64_t n);
hipError_t launch_argmax(const float* x, uint64_t n, uint32_t* out, void* scratch, hipStream_t s);

// Raw GGUF bytes -> tile layout.
hipError_t launch_repack(const void* raw, const TileGeom& g, uint4* recs, uint16_t* dvals, hipStream_t s);

// x [n_vec][cols] (row stride x_stride floats) -> digits + scales; columns in
// [cols, cols_pad) are written as zero. wide: one scale per 256 columns,
// repeated in the unit's eight block slots (cols_pad a multiple of 256; the
// grouped IQ2_XXS matmul requires it).
hipError_t launch_quantize(const float* x, uint64_t x_stride, uint32_t n_vec, uint32_t cols,
                           uint32_t cols_pad, const QuantAct& q, hipStream_t s, bool wide = false);

// Quantised-weight GEMV over n_probs matrices in one launch (activations are
// quantised inside the kernel).
hipError_t launch_gemv_q(const GemvArgs& a, uint32_t fmt, int num_cu, hipStream_t s);
// Up to kGemvMaxSegs such GEMVs of one format in ONE launch: segments may
// differ in weight, shape, activations and outputs (e.g. a layer's experts'
// gate/up and down projections). Segment s is grid slice blockIdx.z = s and
// problem p of it grid row p (rows past its n_probs exit at once), so a
// workgroup finds its arguments without reading any first. Not for
// route_decode.
constexpr uint32_t kGemvMaxSegs = 4;
template <int N>
struct GemvSet {
    GemvArgs seg[N];
};
hipError_t launch_gemv_segments(const GemvArgs* segs, uint32_t n_segs, uint32_t fmt, int num_cu, hipStream_t s);
// IQ2_XXS decode GEMV (gemv_iq2.hip); launch_gemv_q / launch_gemv_segments
// forward IQ2_XXS here.
hipError_t launch_gemv_iq2(const GemvArgs* segs, uint32_t n_segs, int num_cu, hipStream_t s);

// Decode (one token) down projection of the computed experts and the
// combine, IQ2_XXS experts with the shared expert merged (or none): problem
// p of probs[0, *n_active) is {matrix, activation slot, output slot, 0};
// its input is silu(x[slot]) * x[slot] + x2_off (rows x_stride floats
// apart). out = the combined token (combine_kernel's sum).
struct DownCombineArgs {
    const uint4* recs;
    const uint16_t* dvals;
    uint64_t rec_stride, d_stride;
    uint32_t d_row;
    const uint4* probs;
    const uint32_t* n_active;
    const float* x;
    uint64_t x_stride, x2_off;
    const int32_t* assign_slot;
    const float* assign_w;
    const int32_t* shared_slot;
    const uint32_t* deferred;
    const float* bias;              // or null
    float* out;
    uint32_t tiles, units, rows, cols;
};
hipError_t launch_down_combine_iq2(const DownCombineArgs& a, hipStream_t s);

// One-launch decode MoE layer for IQ2_XXS experts (decode_moe.hip): router,
// routing, gate/up, down and combine of one token in one cooperative launch
// of num_cu workgroups. Matrices: gate e / up E + e / shared gate 2E / shared
// up 2E + 1 in gu_*, down e / shared down E in dn_*.
struct DecodeMoeArgs {
    RouteArgs route;            // n_tokens 1; scores: the router's output [E]
    const void* router_w;       // [E][hidden], f32 (router_type 0) or f16 (1)
    uint32_t router_type;
    const float* x;             // hidden vector [hidden]
    uint32_t hidden, inter;     // multiples of 256, at most 2048
    const uint4* gu_recs;
    const uint16_t* gu_dvals;
    uint64_t gu_rec_stride, gu_d_stride;
    uint32_t gu_d_row;
    const uint4* dn_recs;
    const uint16_t* dn_dvals;
    uint64_t dn_rec_stride, dn_d_stride;
    uint32_t dn_d_row;
    uint8_t* hq;                // [5][inter / 32][64] digit planes of silu(gate) * up
    float* hs;                  // [5][inter / 32] their block scales
    uint64_t* score_tags;       // [n_experts] (epoch << 32 | score bits), published by the router rows
    uint32_t* h_flags;          // [5][inter / 32] epoch of the call whose h block is published
    uint32_t epoch;             // this call's number, never 0; the buffers above start zeroed
    uint32_t wait_ticks;        // 10 ns ticks after its first poll before a grid wait gives up
    uint32_t* status;           // host-visible word: nonzero when a grid wait timed out
    const float* bias;          // deferral bias [hidden] or null
    float* out;                 // [hidden]
};
bool decode_moe_iq2_fits(uint32_t hidden, uint32_t inter, uint32_t n_experts, int num_cu);
// Default bound of one grid-wide wait: 10 ms, far beyond a launch whose
// workgroups are all resident (its waits take microseconds).
constexpr uint32_t kDecodeWaitUs = 10000;
hipError_t launch_decode_moe_iq2(const DecodeMoeArgs& a, int num_cu, hipStream_t s);

// Allocation-free QMM scratch (noalloc.hip): kNoallocScratchBytes of device
// memory per device, kept until the process ends. noalloc_scratch() returns
// this device's address; call it with `device` current. Every call on a
// device shares the same bytes.
constexpr size_t kNoallocScratchBytes = 4456448;  // quantised activations of 256 vectors x 8192 columns
hipError_t noalloc_scratch(int device, void** out);

// Plain f32 / f16 weight GEMV (router, matVecMulUnified's f32 branch):
// y_i = W_{first+i} . x_i for i < n_mats.
hipError_t launch_gemv_float(const void* w, uint32_t ggml_type, uint64_t mat_stride,
                             const float* x, uint64_t x_stride, float* y, uint64_t y_stride,
                             uint32_t n_mats, uint32_t rows, uint32_t cols, hipStream_t s);

// Quantised matmul over items of <= 8 activation rows (group.hip).
// Dense: Y = X . W^T for `batch` rows; out_layout 0: y[b * y_ld + r],
// 1: y[r * y_ld + b].
hipError_t launch_group_dense(const uint4* recs, const uint16_t* dvals, const TileGeom& g, uint64_t mat,
                              const QuantAct& xq, uint32_t batch, float* y, uint64_t y_ld, int out_layout,
                              int num_cu, hipStream_t s);
// Dense Q8_0 in one launch (the activations quantised inside, each tile's K
// range split over waves): Y = X . W^T as launch_group_dense computes it
// from launch_quantize's output, for the shapes qmm_q8_fused_fits accepts
// (K <= 2048 columns). x rows are x_stride floats apart; columns >= cols
// read as zero.
bool qmm_q8_fused_fits(const TileGeom& g);
hipError_t launch_qmm_q8_fused(const uint4* recs, const uint16_t* dvals, const TileGeom& g, uint64_t mat,
                               const float* x, uint64_t x_stride, uint32_t cols, uint32_t batch, float* y,
                               uint64_t y_ld, int out_layout, hipStream_t s);
// Grouped: item i < *n_work multiplies activation rows a_row[slot ..
// slot + count) (a_row null: the slots themselves) by matrix work[i].mat and
// writes y[(slot + j) * y_ld + pad + r]. max_work bounds the grid.
hipError_t launch_group_experts(const uint4* recs, const uint16_t* dvals, const TileGeom& g, const QuantAct& xq,
                                const uint32_t* a_row, const QmmWork* work, const uint32_t* n_work, uint32_t max_work,
                                float* y, uint64_t y_ld, int num_cu, hipStream_t s);

// Quantises silu(g) * u per row (rows r < *n_rows, or n_rows_max when
// n_rows is null): g = src + r * src_stride, u = g + u_off.
hipError_t launch_quantize_silu(const float* src, uint64_t src_stride, uint64_t u_off, const uint32_t* n_rows,
                                uint32_t n_rows_max, uint32_t cols, uint32_t cols_pad, const QuantAct& q,
                                hipStream_t s, bool wide = false);

// ---- MoE routing and combine (moe.hip) ----
//
// Activation slots of one MoE call over T tokens: routed (token, expert)
// pairs occupy slots [0, 4T) (T == 1: route order; T > 1: sorted by expert,
// tokens in order), the shared expert of token t is slot 4T + t. Gate/up
// outputs are rows of 2 * inter floats per slot (gate, then up), expert
// outputs rows of hidden floats.

// Scheduler.route (scheduler.zig:169-262) for every token on the device, plus
// the problem lists of the expert products.

hipError_t launch_route(const RouteArgs& a, hipStream_t s);
// Upper bound of the grouped items per list for T tokens and E experts.
uint32_t route_max_work(uint32_t n_tokens, uint32_t n_experts);

// out[t] = sum over the token's routed slots, in route order, of w * eo[slot]
// (products and sums rounded separately), + eo[shared slot], + bias when
// deferred  (moeFFN, inference.zig:977-1006).
hipError_t launch_combine(const float* eo, const int32_t* assign_slot, const float* assign_w,
                          const int32_t* shared_slot, const uint32_t* deferred, const float* bias, float* out,
                          uint32_t n_tokens, uint32_t hidden, hipStream_t s);

}  // namespace mmhip
