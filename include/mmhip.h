/*
 * libmmhip: MI355X (gfx950) backend for the quantized-weight matrix path of
 * mobile-moe.zig — Q8_0 / IQ2_XXS dequantisation, decode GEMV, batched QMM
 * and the MoE expert FFN — behind a plain C ABI.
 *
 * Conventions follow the reference's C bridge (src/metal_bridge.c:50-87,
 * src/metal_backend.zig:7-46): opaque handles, int status (0 = ok, < 0 =
 * error), and a last-error string. The error string is thread-local here
 * because the reference re-enters its seam from 4 pool workers
 * (src/inference.zig:934-971).
 *
 * Pointers named *_host are ordinary host memory; pointers named *_dev are
 * device memory (e.g. from mmhip_malloc). Every *_dev entry point is
 * asynchronous on the context's stream (mmhip_stream); every host-slice
 * entry point is synchronous, like OpenCLBackend's calls that end in
 * clFinish (src/opencl_backend.zig:452).
 *
 * Tensor types use GgmlType ids (src/gguf.zig:21-56). Quantised weights are
 * passed as raw GGUF bytes: Q8_0 blocks {f16 d; i8 qs[32]} (34 B,
 * src/dequant.zig:372-377) and IQ2_XXS superblocks {f16 d; u16 qs[32]}
 * (66 B, src/dequant.zig:305-311), row-major, rows of ceil(cols/bs) blocks.
 * Uploading converts them once into the device tile layout the kernels read;
 * the bytes per block stay the same.
 *
 * There is no CPU fallback anywhere in this library: without a usable HIP
 * device every compute entry point returns MMHIP_ERR_UNAVAILABLE. The
 * caller's engine decides what to do then (the reference falls back to its
 * own CPU kernels at src/inference.zig:1209-1213).
 */
#ifndef MMHIP_H
#define MMHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---- */
#define MMHIP_OK 0
#define MMHIP_ERR_UNAVAILABLE (-1) /* no HIP device / runtime */
#define MMHIP_ERR_INVALID (-2)     /* bad argument or shape */
#define MMHIP_ERR_UNSUPPORTED (-3) /* tensor type not on this path */
#define MMHIP_ERR_HIP (-4)         /* HIP runtime error (see last error) */
#define MMHIP_ERR_NOMEM (-5)
#define MMHIP_ERR_NOT_FOUND (-6) /* GGUF tensor or metadata key absent, or of another type */

/* ---- GgmlType ids (src/gguf.zig:21-56) ---- */
#define MMHIP_TYPE_F32 0u
#define MMHIP_TYPE_F16 1u
#define MMHIP_TYPE_Q8_0 8u
#define MMHIP_TYPE_IQ2_XXS 16u

typedef struct mmhip_ctx mmhip_ctx;
typedef struct mmhip_weight mmhip_weight;
typedef struct mmhip_moe_layer mmhip_moe_layer;

/* ======================================================================
 * Backend object: replaces OpenCLBackend's lifecycle
 * (src/opencl_backend.zig:92-300) and metal_init / metal_get_last_error
 * (src/metal_bridge.c:52-87).
 * ====================================================================== */

/* Last error message of the calling thread ("" if none). */
const char* mmhip_last_error(void);
/* 1 if a gfx950 device is usable (OpenCLBackend.isAvailable, 92-99). */
int mmhip_is_available(void);
/* Number of visible HIP devices (0 if the runtime is absent). */
int mmhip_device_count(void);
/* Library build identifier (static string). */
const char* mmhip_version(void);

/* OpenCLBackend.init (101-281): create a context on `device`. */
int mmhip_init(mmhip_ctx** out_ctx, int device);
/* OpenCLBackend.deinit (283-300): frees every resident weight. */
void mmhip_destroy(mmhip_ctx* ctx);
/* Wait for all work queued on the context's stream (clFinish). Also reports
 * a failed grid-wide wait of an earlier one-launch MoE decode
 * (mmhip_moe_ffn_dev): MMHIP_ERR_HIP with the reason, once, and the status
 * is cleared. A caller that synchronises the raw stream from mmhip_stream()
 * instead never sees that error. */
int mmhip_synchronize(mmhip_ctx* ctx);
/* The context's hipStream_t, as an opaque pointer. */
void* mmhip_stream(mmhip_ctx* ctx);
/* Number of compute units of the context's device. */
int mmhip_num_cu(mmhip_ctx* ctx);

/* Kernel timing: when enabled, HIP events are recorded on the context's
 * stream around every launch of the hot kernels; mmhip_profile_read sums
 * them per kernel family ("gemv_q", "gemv_float", "qmm", "quantize",
 * "moe_router", "moe_route", "moe_quantize", "moe_gateup", "moe_down", "moe_decode",
 * "moe_combine"). This fills the role
 * of the per-op GPU timings the reference leaves empty
 * (op_perf_db.zig:88-97). Enabling resets the accumulators. */
int mmhip_profile_enable(mmhip_ctx* ctx, int enable);
int mmhip_profile_read(mmhip_ctx* ctx, const char* family, double* total_ms, uint64_t* launches);

/* Device memory helpers, so callers need no other HIP binding. */
int mmhip_malloc(mmhip_ctx* ctx, void** out_dev, size_t bytes);
int mmhip_free(mmhip_ctx* ctx, void* dev);
int mmhip_memcpy_h2d(mmhip_ctx* ctx, void* dst_dev, const void* src_host, size_t bytes);
int mmhip_memcpy_d2h(mmhip_ctx* ctx, void* dst_host, const void* src_dev, size_t bytes);
int mmhip_memset_dev(mmhip_ctx* ctx, void* dst_dev, int value, size_t bytes);

/* ======================================================================
 * Device-resident weights: replaces getOrUploadMatBuffer's residency cache
 * (src/opencl_backend.zig:311-323) with explicit handles.
 * `count` stacks matrices of [rows x cols] back to back, as the expert
 * tensors ffn_{gate,up,down}_exps are stored ([n_experts][rows][cols],
 * src/inference.zig:1148-1166).
 * One repacked Q8_0 / IQ2_XXS matrix must stay below 2 GiB (about 2e9
 * Q8_0 weights); a larger one is MMHIP_ERR_UNSUPPORTED. `count` is not
 * limited by this.
 * ====================================================================== */

int mmhip_weight_upload(mmhip_ctx* ctx, const void* raw_host, uint32_t type,
                        uint64_t rows, uint64_t cols, uint64_t count,
                        mmhip_weight** out_w);
/* Same, from raw GGUF bytes already in device memory (not retained). */
int mmhip_weight_from_device(mmhip_ctx* ctx, const void* raw_dev, uint32_t type,
                             uint64_t rows, uint64_t cols, uint64_t count,
                             mmhip_weight** out_w);
void mmhip_weight_free(mmhip_ctx* ctx, mmhip_weight* w);
/* Device bytes held by the weight (tile records + scales). */
uint64_t mmhip_weight_device_bytes(const mmhip_weight* w);

/* ======================================================================
 * GGUF v3 files and device-resident weights from them. These replace
 *   gguf.loadFromFile / parse (src/gguf.zig:266-413): the file is mapped
 *     read-only (MAP_PRIVATE + MADV_WILLNEED) and parsed; errors carry the
 *     reference's names (InvalidMagic, UnsupportedVersion, StringTooLong,
 *     ArrayTooLong, TooManyDimensions, UnsupportedMetadataType,
 *     UnsupportedArrayType, EndOfStream) in mmhip_last_error();
 *   GgufFile.tensor_infos.get + tensorPtr (src/gguf.zig:218-229);
 *   GgufFile.metaString / metaInt / metaFloat (src/gguf.zig:232-262);
 *   Model.bindTensor / bindLayer's FFN tensors (src/model.zig:261-395) with
 *     a one-time upload into the tile layout the kernels read.
 * A tensor's dims[0] is its row length (ggml order): a matrix stack is
 * [cols, rows, count]. Pointers returned stay valid until mmhip_gguf_close.
 * ====================================================================== */

typedef struct mmhip_gguf mmhip_gguf;
typedef struct {
    uint32_t version;            /* 3 */
    uint64_t tensor_count;       /* header counts */
    uint64_t metadata_count;
    uint64_t n_tensors, n_keys;  /* distinct names / keys */
    uint64_t alignment;          /* general.alignment or 32 */
    uint64_t data_offset;        /* start of the tensor data section */
    uint64_t file_size;
} mmhip_gguf_info;
typedef struct {                 /* TensorInfo (src/gguf.zig:162-175) */
    const char* name;
    uint32_t n_dims;
    uint64_t dims[4];            /* unused dimensions are 1 */
    uint32_t type;               /* GgmlType */
    uint64_t offset;             /* from data_offset */
    uint64_t n_elements;         /* TensorInfo.nElements */
    uint64_t n_bytes;            /* GgmlType.tensorBytes; 0 for a type this library does not read */
    const void* data;            /* mapped bytes, NULL if the type is not read here or they leave the file */
} mmhip_gguf_tensor;

int mmhip_gguf_open(const char* path, mmhip_gguf** out);
void mmhip_gguf_close(mmhip_gguf* g);
int mmhip_gguf_get_info(const mmhip_gguf* g, mmhip_gguf_info* out);
/* Tensors and keys in file order (first occurrence of a repeated name). */
int mmhip_gguf_tensor_at(const mmhip_gguf* g, uint64_t index, mmhip_gguf_tensor* out);
int mmhip_gguf_find_tensor(const mmhip_gguf* g, const char* name, mmhip_gguf_tensor* out);
const char* mmhip_gguf_key_at(const mmhip_gguf* g, uint64_t index);
/* Metadata value type (MetadataValueType, src/gguf.zig:121-135) or < 0. */
int mmhip_gguf_meta_type(const mmhip_gguf* g, const char* key);
int mmhip_gguf_meta_int(const mmhip_gguf* g, const char* key, int64_t* out);
int mmhip_gguf_meta_float(const mmhip_gguf* g, const char* key, double* out);
/* Not NUL-terminated: *len bytes. */
int mmhip_gguf_meta_string(const mmhip_gguf* g, const char* key, const char** str, uint64_t* len);
/* Numeric arrays: len little-endian elements; string arrays: len records of
 * [u64 length][bytes] (the layout MetadataArray.data holds). */
int mmhip_gguf_meta_array(const mmhip_gguf* g, const char* key, uint32_t* elem_type, uint64_t* len,
                          const void** data, uint64_t* n_bytes);
/* mmhip_weight_upload of the named tensor (rows = dims[1], cols = dims[0],
 * count = dims[2]). */
int mmhip_weight_upload_gguf(mmhip_ctx* ctx, const mmhip_gguf* g, const char* name, mmhip_weight** out_w);
/* One weight whose rows are the named matrices' rows stacked in order (same
 * type and row length, one matrix each), e.g. attn_q_a then attn_kv_a_mqa,
 * which read the same hidden vector (src/inference.zig:467-489): one GEMV
 * launch gives both projections. */
int mmhip_weight_upload_gguf_rows(mmhip_ctx* ctx, const mmhip_gguf* g, const char* const* names, uint32_t n,
                                  mmhip_weight** out_w);
/* mmhip_moe_layer_create from blk.<layer>.ffn_gate_inp / ffn_{gate,up,down}_exps
 * and, when present, ffn_{gate,up,down}_shexp (the shared width is their
 * row count); routed_scaling_factor from deepseek2.expert_weights_scale
 * (default 1), the key HyperParams.fromGguf reads (model.zig:107). */
int mmhip_moe_layer_create_gguf(mmhip_ctx* ctx, const mmhip_gguf* g, uint32_t layer,
                                mmhip_moe_layer** out_layer);

/* ======================================================================
 * Engine seam, host slices. These replace the bodies of
 *   matVecMulUnified   (src/inference.zig:1200-1228)
 *   batchMatMulUnified (src/inference.zig:1231-1264)
 *   dequant.dequantize (src/dequant.zig:632-659)
 * and OpenCLBackend.matMulQ8_0 (src/opencl_backend.zig:412-453). The weight
 * is uploaded on first use and kept resident, keyed by (ptr, type, shape).
 * Supported types: F32, F16, Q8_0, IQ2_XXS.
 * ====================================================================== */

int mmhip_mat_vec_mul(mmhip_ctx* ctx, float* out_host, const void* ptr_host,
                      uint32_t type, const float* x_host, uint64_t out_dim,
                      uint64_t in_dim);
/* out [batch][out_dim] = in [batch][in_dim] . W^T (the seam's layout). */
int mmhip_batch_mat_mul(mmhip_ctx* ctx, float* out_host, const void* ptr_host,
                        uint32_t type, const float* in_host, uint64_t out_dim,
                        uint64_t batch, uint64_t in_dim);
int mmhip_dequantize(mmhip_ctx* ctx, float* out_host, const void* data_host,
                     uint32_t type, uint64_t n_elements);
/* quantizeQ8_0 (dequant.zig:98-130): n floats -> ceil(n / 32) raw Q8_0
 * blocks of 34 bytes (per block: d = max|x| / 127 stored as f16, q = x / d
 * rounded half away from zero, clamped to +-127; the last block padded with
 * zeros). Bit-exact with the CPU path except on the f16 subnormal range of
 * the block scale, d in [2^-25, 2^-14), where the reference's f32ToF16
 * (dequant.zig:76-77) shifts the significand by 1 - exp16: for d in
 * [2^-21, 2^-14) its @intCast traps, and for d in [2^-25, 2^-21) it returns a
 * corrupted code (e.g. d = 2^-22 -> 0x8000, d = 1.5 * 2^-23 -> 0x6000). Here
 * the scale on that whole range is the subnormal value truncated toward
 * zero (d = 2^-22 -> 0x0004). A NaN value quantises to 0. */
int mmhip_quantize_q8_0(mmhip_ctx* ctx, void* blocks_host, const float* x_host,
                        uint64_t n_elements);
/* sampleGreedy (inference.zig:376-386) over n logits (computeLogits'
 * output, inference.zig:1189-1197): *out_host = the first index of the
 * largest logit (strict >, so ties keep the earlier index; a NaN never
 * wins; a NaN logits[0] gives 0). 1 <= n < 2^32. */
int mmhip_sample_greedy(mmhip_ctx* ctx, uint32_t* out_host, const float* logits_host,
                        uint64_t n);
/* Drop the resident copy keyed by ptr_host (all types/shapes). */
int mmhip_forget(mmhip_ctx* ctx, const void* ptr_host);

/* ======================================================================
 * Device twins (asynchronous on mmhip_stream(ctx)).
 * ====================================================================== */

/* dequantize from raw GGUF bytes in device memory; bit-exact. */
int mmhip_dequantize_dev(mmhip_ctx* ctx, float* out_dev, const void* raw_dev,
                         uint32_t type, uint64_t n_elements);
/* KVCache.put's Q8_0 branch (kv_cache.zig:289-349) for n_rows positions at
 * once: row r of row_len floats (x_dev + r * x_stride) -> ceil(row_len / 32)
 * blocks at blocks_dev + r * ceil(row_len / 32) * 34, as mmhip_quantize_q8_0
 * per row. blocks_dev must be 4-byte aligned. */
int mmhip_quantize_q8_0_rows_dev(mmhip_ctx* ctx, void* blocks_dev, const float* x_dev,
                                 uint64_t x_stride, uint64_t n_rows, uint32_t row_len);
/* getKVCompressed / getKPe's Q8_0 branch (kv_cache.zig:225-273) for n_rows
 * positions: out_dev[r * out_stride + c] = f16ToF32(d) * q; bit-exact.
 * blocks_dev must be 2-byte aligned. */
int mmhip_dequantize_q8_0_rows_dev(mmhip_ctx* ctx, float* out_dev, uint64_t out_stride,
                                   const void* blocks_dev, uint64_t n_rows, uint32_t row_len);
/* mmhip_sample_greedy on device logits; *out_dev receives the token id. The
 * logits come from mmhip_gemv_dev with the output projection weight
 * (computeLogits: hidden -> vocab_size). */
int mmhip_argmax_dev(mmhip_ctx* ctx, uint32_t* out_dev, const float* logits_dev, uint64_t n);
/* y[rows] = W[mat] . x[cols] for one matrix of a weight. */
int mmhip_gemv_dev(mmhip_ctx* ctx, const mmhip_weight* w, uint64_t mat,
                   const float* x_dev, float* y_dev);
/* n_mats products in ONE launch: y_i = W[first + i] . x_i with
 * x_i = x_dev + i * x_stride, y_i = y_dev + i * y_stride (strides in
 * floats; x_stride 0 shares one input vector). */
int mmhip_gemv_batched_dev(mmhip_ctx* ctx, const mmhip_weight* w,
                           uint64_t first, uint64_t n_mats,
                           const float* x_dev, uint64_t x_stride,
                           float* y_dev, uint64_t y_stride);
/* Several mmhip_gemv_batched_dev calls in ONE launch: each group is a range
 * of matrices of its own weight (weights may differ in shape, not in type;
 * Q8_0 or IQ2_XXS), with its own inputs and outputs (strides in floats, 0
 * shares one input vector). No counterpart in the reference: it issues the
 * matVecMulUnified calls of a layer's experts (expertFFN,
 * inference.zig:1171-1185), e.g. the routed experts' gate/up [1536 x 2048]
 * and down [2048 x 1536] products of a step, as one launch instead of one per
 * shape. IQ2_XXS results equal the separate calls' bit for bit; Q8_0 results
 * agree to f32 rounding (a tile's record units may be split over the waves
 * differently). */
#define MMHIP_GEMV_MAX_GROUPS 4u
typedef struct {
    const mmhip_weight* w;
    uint64_t first, n_mats;
    const float* x_dev;
    uint64_t x_stride;
    float* y_dev;
    uint64_t y_stride;
} mmhip_gemv_group;
int mmhip_gemv_grouped_dev(mmhip_ctx* ctx, const mmhip_gemv_group* groups, uint32_t n_groups);
/* Batched QMM for prompt prefill: X [batch][cols] -> Y.
 * out_layout 0: Y [batch][rows] (batchMatMulUnified's layout);
 * out_layout 1: Y [rows][batch] (qmm.matMulQ8_0's layout, qmm.zig:52-57). */
int mmhip_qmm_dev(mmhip_ctx* ctx, const mmhip_weight* w, uint64_t mat,
                  const float* x_dev, float* y_dev, uint64_t batch,
                  int out_layout);

/* mmhip_qmm_dev without any allocation, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, hosts
 * that forbid hipMalloc). No counterpart in the reference. Same kernels and
 * results as mmhip_qmm_dev; the quantised activations go to a fixed scratch
 * of MMHIP_NOALLOC_SCRATCH_BYTES per device, held until the process ends, so
 * quantised weights need batch x cols256 x 2.125 <= MMHIP_NOALLOC_SCRATCH_BYTES
 * (cols256 = cols rounded up to 256: e.g. 256 rows of 8192 columns), else
 * MMHIP_ERR_INVALID. Calls on one device share that scratch: calls that
 * overlap on a device (two streams, two contexts, two threads) race. Not
 * timed by mmhip_profile_*. f32 / f16 weights use no scratch, nor do Q8_0
 * weights of at most 2048 columns (their activations are quantised inside
 * the one matmul launch; MMHIP_QMM_FUSED=0 turns that off). */
#define MMHIP_NOALLOC_SCRATCH_BYTES 4456448u
int mmhip_qmm_dev_noalloc(mmhip_ctx* ctx, const mmhip_weight* w, uint64_t mat,
                          const float* x_dev, float* y_dev, uint64_t batch,
                          int out_layout);

/* ======================================================================
 * MoE FFN layer: replaces moeFFN (src/inference.zig:886-1010) with
 * expertFFN (1152-1188), sharedExpertFFN (1094-1146), Scheduler.route
 * (src/scheduler.zig:169-262) and the per-token batch loop of forwardBatch
 * (src/inference.zig:346-351). Routing, expert FFNs, the weighted sum and
 * the shared expert all run on the device; nothing is copied back between
 * steps.
 * ====================================================================== */

typedef struct {
    uint32_t hidden_size;          /* hp.hidden_size (2048) */
    uint32_t moe_intermediate;     /* hp.moe_intermediate_size (1536) */
    uint32_t shared_intermediate;  /* width of the shared expert */
    uint32_t n_routed_experts;     /* hp.n_routed_experts (64) */
    uint32_t expert_type;          /* lw.expert_type (Q8_0 or IQ2_XXS) */
    uint32_t shared_type;          /* lw.shared_type */
    uint32_t router_type;          /* lw.moe_gate_type (F32 or F16) */
    float routed_scaling_factor;   /* hp.routed_scaling_factor */
    const void* router_host;       /* [n_experts][hidden] */
    const void* expert_gate_host;  /* [n_experts][moe_inter][hidden] */
    const void* expert_up_host;    /* [n_experts][moe_inter][hidden] */
    const void* expert_down_host;  /* [n_experts][hidden][moe_inter] */
    const void* shared_gate_host;  /* [shared_inter][hidden], NULL = none */
    const void* shared_up_host;
    const void* shared_down_host;  /* [hidden][shared_inter] */
} mmhip_moe_weights;

/* Throttle inputs of Scheduler.route (ThrottleState fields,
 * src/thermal.zig:17-72). level: 0 normal, 1 light, 2 medium, 3 heavy. */
typedef struct {
    int32_t throttle_level;
    uint32_t active_expert_limit;  /* 0 = the level's default (4/3/2/1) */
    const float* deferral_bias_host; /* [hidden] or NULL (Scheduler.deferral_bias) */
} mmhip_route_params;

#define MMHIP_MOE_MAX_TOKENS 256u  /* forwardBatch's max_batch_size (inference.zig:115) */

int mmhip_moe_layer_create(mmhip_ctx* ctx, const mmhip_moe_weights* wts,
                           mmhip_moe_layer** out_layer);
void mmhip_moe_layer_destroy(mmhip_ctx* ctx, mmhip_moe_layer* layer);

/* n_tokens hidden vectors in, n_tokens FFN outputs out (host buffers,
 * synchronous). route_ids / route_weights (optional, [n_tokens][4]) receive
 * Scheduler.route's expert_ids / weights; unused slots hold 0xFFFFFFFF / 0.
 * Returns k (experts per token) or < 0.
 *
 * One-token calls on a layer with IQ2_XXS experts (shared expert merged or
 * absent) run as ONE launch whose workgroups (one per CU) hand work to each
 * other, so all of them must be resident at once. That holds while no other
 * kernel occupies the device's CUs (another stream, context or process);
 * one that does delays the launch until its CUs free up. A hand-over wait
 * that is not satisfied within 10 ms (MMHIP_DECODE_WAIT_US) gives up: the
 * launch still ends, its output is invalid, and the error is returned by
 * this call, or, for mmhip_moe_ffn_dev, by the next mmhip_synchronize or
 * mmhip_moe_ffn on the context. MMHIP_DECODE_FUSED=0 (read at layer
 * creation) selects three ordinary launches, which need no residency, and
 * MMHIP_DECODE_COOP=1 a cooperative launch, which guarantees it (~18 us
 * more per call). */
int mmhip_moe_ffn(mmhip_ctx* ctx, mmhip_moe_layer* layer, const float* hidden_host,
                  float* out_host, uint32_t n_tokens, const mmhip_route_params* rp,
                  uint32_t* route_ids_host, float* route_weights_host);
/* Device twin (asynchronous). route_*_dev may be NULL. Returns 0 or < 0;
 * a failed hand-over wait of its one-launch decode (above) is reported by
 * the next mmhip_synchronize or mmhip_moe_ffn, after work queued behind it
 * may already have read the invalid output. */
int mmhip_moe_ffn_dev(mmhip_ctx* ctx, mmhip_moe_layer* layer, const float* hidden_dev,
                      float* out_dev, uint32_t n_tokens, const mmhip_route_params* rp,
                      uint32_t* route_ids_dev, float* route_weights_dev);
/* ExpertStats.counts for this layer (scheduler.zig:19-44): activations per
 * expert since creation, [n_routed_experts]. Synchronous. */
int mmhip_moe_expert_counts(mmhip_ctx* ctx, mmhip_moe_layer* layer, uint64_t* counts_host);

/* ======================================================================
 * Operator planner: OpScheduler / LayerPlan (src/scheduler.zig:265-552)
 * with the GPU rules this backend adds. Host logic only; no device needed.
 * ====================================================================== */

/* op_perf_db.OpType (src/op_perf_db.zig:26-40) */
enum {
    MMHIP_OP_MATMUL_Q8_0 = 0, MMHIP_OP_MATMUL_Q4_K, MMHIP_OP_MATMUL_F32,
    MMHIP_OP_MATVEC_Q8_0, MMHIP_OP_MATVEC_F32, MMHIP_OP_RMSNORM,
    MMHIP_OP_SILU_MUL, MMHIP_OP_ROPE, MMHIP_OP_SOFTMAX, MMHIP_OP_DOT,
    MMHIP_OP_ATTENTION, MMHIP_OP_FFN_GATE_UP, MMHIP_OP_FFN_DOWN
};
/* op_perf_db.Precision (43-48) plus the iq2_xxs value this backend adds. */
enum { MMHIP_PREC_Q8_0 = 0, MMHIP_PREC_Q4_K, MMHIP_PREC_F32, MMHIP_PREC_F16, MMHIP_PREC_IQ2_XXS };
/* scheduler.Backend (268-272) */
enum { MMHIP_BACKEND_CPU = 0, MMHIP_BACKEND_GPU = 1, MMHIP_BACKEND_NPU = 2 };

typedef struct { uint32_t m, n, k, dim; } mmhip_shape;          /* op_perf_db.Shape */
typedef struct {                                                /* OpSchedule (275-288) */
    uint32_t op, backend, precision, sync_after;
    mmhip_shape shape;
    uint64_t estimated_us;
} mmhip_op_schedule;
typedef struct {                                                /* PlanHyperParams (544-552) */
    uint32_t hidden_size, intermediate_size, num_heads, head_dim;
    uint32_t seq_len_hint;          /* 0 = 128 */
    uint32_t leading_dense_layers, n_routed_experts;
    uint32_t weight_precision;      /* MMHIP_PREC_* of the FFN weights */
} mmhip_plan_hparams;
typedef struct {                                                /* OpPerfDb entry (88-97) */
    uint32_t op, precision;
    mmhip_shape shape;
    uint64_t cpu_us, gpu_us;
} mmhip_perf_entry;

/* OpScheduler.init + planLayer (364-503). has_gpu normally comes from
 * mmhip_is_available(). Writes up to `cap` schedules, *n_out = count. */
int mmhip_plan_layer(uint32_t layer, const mmhip_plan_hparams* hp, int has_gpu,
                     int has_npu, int throttle_level, const mmhip_perf_entry* db,
                     size_t db_len, mmhip_op_schedule* out, size_t cap, size_t* n_out);
/* LayerPlan.estimatedCriticalPathUs (313-333) */
uint64_t mmhip_plan_critical_path_us(const mmhip_op_schedule* ops, size_t n);
/* LayerPlan.deviceMask (336-346) */
uint32_t mmhip_plan_device_mask(const mmhip_op_schedule* ops, size_t n);

#ifdef __cplusplus
}
#endif
#endif
