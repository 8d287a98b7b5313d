/*
 * CPU oracle for the quantized-matrix / MoE-FFN path of mobile-moe.zig.
 *
 * TEST INFRASTRUCTURE ONLY. This is a plain-C restatement of the reference's
 * CPU algorithm (Zig 0.16, which cannot be built in this environment). Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it,
 * and only as the checker / the timed CPU baseline. The HIP library never
 * links or calls it.
 *
 * Every function names the reference lines it follows. Floating-point
 * evaluation order follows the reference: 4-lane vector accumulators reduced
 * lane 0..3 in order (Zig @reduce(.Add) in strict float mode is an ordered
 * reduction), products and sums never contracted into FMAs (the build uses
 * -ffp-contract=off, matching Zig's default strict float mode).
 *
 * Pinning (what checks each function; see tests/test_oracle_*.py):
 *   orc_f16_to_f32          reference KATs dequant.zig:663-707 + exhaustive
 *                           65,536-code comparison with IEEE binary16->32.
 *   orc_f32_to_f16          reference KATs (1.0, 2.0, 0.5, 1/127) + numpy RNE
 *                           on the normal range; the subnormal branch is a
 *                           reference defect (see the function): *defect = 1
 *                           where the reference traps, 2 where it returns a
 *                           corrupted code, pinned by hand-derived codes.
 *   orc_dequantize_q8_0     closed form d*q (exact in f32) on all 65,536 d codes.
 *   orc_sample_greedy       numpy argmax (first occurrence) on NaN-free data,
 *                           hand-derived cases: ties, -0 vs +0, NaN at 0 and
 *                           elsewhere, all equal, -inf.
 *   orc_quantize_q8_0       reference KAT kv_cache.zig:686-719 (put/get round
 *                           trip within 5% + 1e-2), stored d = f32ToF16(max/127)
 *                           (normal range: the pinned converter; subnormal:
 *                           exact integer truncation), q = the nearest integer
 *                           to x/d with ties away from zero (searched over
 *                           [-127, 127]), +-127 at each block's largest |x|,
 *                           zero blocks and padding.
 *   orc_dequantize_iq2xxs   hand-derived special cases (all-zero block = 1.0,
 *                           byte order of grid entries, sign bit positions,
 *                           ls=15 scale), codebook invariants, ksigns closed form.
 *   orc_matvec_q8_0         reference KAT qmm.zig:213-238, f64 dot products.
 *   orc_matmul_q8_0         reference KATs qmm.zig:142-211, f64 dot products.
 *   orc_matvec_f32 / dot    reference KAT math.zig:284-287, f64 dot products.
 *   orc_topk                reference KAT math.zig:274-282, brute-force sort.
 *   orc_silu                reference KAT math.zig:256-259, closed form.
 *   orc_route               closed-form softmax over the selected logits,
 *                           throttle table thermal.zig:44-72.
 *   orc_moe_ffn             composition of the pinned parts + an independent
 *                           float64 recomputation of the same formula. No
 *                           reference test pins it ("parity unpinned by
 *                           reference tests" beyond that composition).
 */
#ifndef MM_ORACLE_H
#define MM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GgmlType ids (gguf.zig:21-56) used on this path. */
enum { ORC_F32 = 0, ORC_F16 = 1, ORC_Q8_0 = 8, ORC_IQ2_XXS = 16 };

/* Throttle levels (thermal.zig:10-15). */
enum { ORC_NORMAL = 0, ORC_LIGHT = 1, ORC_MEDIUM = 2, ORC_HEAVY = 3 };

/* Route targets (scheduler.zig:130-134). */
enum { ORC_TARGET_GPU = 0, ORC_TARGET_CPU = 1, ORC_TARGET_SKIPPED = 2 };

/* ---- formats (dequant.zig, gguf.zig) ---- */
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float v, int* defect);
uint64_t orc_block_size(uint32_t type);
uint64_t orc_block_bytes(uint32_t type);
uint64_t orc_tensor_bytes(uint32_t type, uint64_t n_elements);
uint64_t orc_iq2xxs_grid(uint32_t idx);
uint8_t orc_ksigns(uint32_t code);
void orc_dequantize_q8_0(const uint8_t* data, uint64_t n_elements, float* out);
void orc_quantize_q8_0(const float* x, uint64_t n_elements, uint8_t* out);
uint32_t orc_sample_greedy(const float* logits, uint64_t n);
void orc_quantize_q8_0_rows(const float* x, uint64_t x_stride, uint64_t n_rows, uint32_t row_len, uint8_t* out);
void orc_dequantize_q8_0_rows(const uint8_t* blocks, uint64_t n_rows, uint32_t row_len, float* out);
void orc_dequantize_iq2xxs_block(const uint8_t* block, float* out256);
void orc_dequantize_iq2xxs(const uint8_t* data, uint64_t n_elements, float* out);
int orc_dequantize(const uint8_t* data, uint32_t type, uint64_t n_elements, float* out);

/* ---- CPU kernels (qmm.zig, math.zig) ---- */
void orc_matvec_q8_0(float* out, const uint8_t* blocks, const float* x,
                     size_t out_dim, size_t in_dim);
void orc_matmul_q8_0(float* out, const uint8_t* a_blocks, const float* b,
                     size_t m, size_t n, size_t k);
void orc_matvec_f32(float* out, const float* w, const float* x,
                    size_t out_dim, size_t in_dim);
float orc_dot(const float* a, const float* b, size_t n);
float orc_silu(float x);
void orc_silu_inplace(float* x, size_t n);
void orc_mul(float* out, const float* a, const float* b, size_t n);
/* Returns k; writes descending (index, score) pairs. */
size_t orc_topk(const float* scores, size_t n, size_t k, uint32_t* idx_out,
                float* score_out);

/* ---- engine seam (inference.zig:1200-1264), CPU branch ---- */
int orc_mat_vec_mul_unified(float* out, const uint8_t* ptr, uint32_t type,
                            const float* x, size_t out_dim, size_t in_dim);
int orc_batch_mat_mul_unified(float* out, const uint8_t* ptr, uint32_t type,
                              const float* in, size_t out_dim, size_t batch,
                              size_t in_dim);

/* ---- routing (scheduler.zig:19-262, thermal.zig:44-72) ---- */
typedef struct {
    uint64_t* counts; /* [n_layers * n_experts] */
    uint32_t n_experts;
    uint32_t n_layers;
    uint64_t total_tokens;
} orc_expert_stats;

typedef struct {
    int level;                  /* ORC_NORMAL.. ORC_HEAVY */
    uint32_t active_expert_limit;
    int hot_experts_on_cpu;
} orc_throttle;

void orc_throttle_set(orc_throttle* t, int level);
/* stats may be NULL (targets then treat every expert as cold). Returns k. */
uint32_t orc_route(orc_expert_stats* stats, uint32_t layer,
                   const orc_throttle* thr, float routed_scaling_factor,
                   const float* gate_scores, uint32_t n_experts,
                   uint32_t* expert_ids, float* weights, int* targets,
                   int* deferred);

/* ---- MoE FFN (inference.zig:886-1188) ---- */
typedef struct {
    uint32_t hidden;            /* hp.hidden_size */
    uint32_t moe_inter;         /* hp.moe_intermediate_size */
    uint32_t shared_inter;      /* width used by sharedExpertFFN */
    uint32_t n_experts;         /* hp.n_routed_experts */
    uint32_t expert_type;       /* lw.expert_type */
    uint32_t shared_type;       /* lw.shared_type */
    uint32_t router_type;       /* lw.moe_gate_type */
    const uint8_t* router;      /* [n_experts][hidden] */
    const uint8_t* expert_gate; /* [n_experts][moe_inter][hidden] */
    const uint8_t* expert_up;
    const uint8_t* expert_down; /* [n_experts][hidden][moe_inter] */
    const uint8_t* shared_gate; /* NULL = no shared expert */
    const uint8_t* shared_up;
    const uint8_t* shared_down;
    float routed_scaling_factor;
    const float* deferral_bias; /* [hidden] or NULL */
} orc_moe_desc;

typedef struct orc_pool orc_pool;
orc_pool* orc_pool_create(int n_threads);
void orc_pool_destroy(orc_pool* p);

/* One token. pool may be NULL (serial; identical numerics). Writes the route
 * (k entries) when ids/weights are non-NULL. Returns k, or <0 on error. */
int orc_moe_ffn(const orc_moe_desc* d, orc_pool* pool,
                orc_expert_stats* stats, uint32_t layer,
                const orc_throttle* thr, const float* hidden_in,
                float* hidden_out, uint32_t* route_ids, float* route_w);

/* forwardBatch's per-token MoE loop (inference.zig:346-351). */
int orc_moe_ffn_batch(const orc_moe_desc* d, orc_pool* pool,
                      orc_expert_stats* stats, uint32_t layer,
                      const orc_throttle* thr, const float* hidden_in,
                      float* hidden_out, uint32_t n_tokens,
                      uint32_t* route_ids, float* route_w);

#ifdef __cplusplus
}
#endif
#endif
