// extern "C" surface of libmmhip (declared in include/mmhip.h): context
// lifecycle, device memory helpers, weight residency, and the engine-seam
// entry points (matVecMulUnified / batchMatMulUnified / dequantize).
#include <cstring>
#include <mutex>
#include <string>

#include "../../include/mmhip.h"
#include "backend.hpp"

static_assert(MMHIP_NOALLOC_SCRATCH_BYTES == mmhip::kNoallocScratchBytes, "scratch size in the header and the library differ");
static_assert(MMHIP_GEMV_MAX_GROUPS == mmhip::kGemvMaxSegs, "group limit in the header and the library differ");

namespace mmhip {
const char* last_error_cstr();
}

using namespace mmhip;

namespace {

int require_ctx(mmhip_ctx* ctx) {
    if (!ctx) {
        set_error(MMHIP_ERR_INVALID, "null context");
        return MMHIP_ERR_INVALID;
    }
    return MMHIP_OK;
}

bool gfx950_present(int* count_out) {
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess) count = 0;
    if (count_out) *count_out = count;
    for (int d = 0; d < count; ++d) {
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, d) == hipSuccess && std::strncmp(prop.gcnArchName, "gfx950", 6) == 0)
            return true;
    }
    return false;
}

// Resident weight for a host pointer (getOrUploadMatBuffer semantics).
int resident_weight(mmhip_ctx* ctx, const void* ptr, uint32_t type, uint64_t rows, uint64_t cols,
                    mmhip_weight** out) {
    auto key = std::make_tuple(ptr, type, rows, cols);
    auto it = ctx->resident.find(key);
    if (it != ctx->resident.end()) {
        *out = it->second;
        return MMHIP_OK;
    }
    int rc = weight_create(ctx, ptr, false, type, rows, cols, 1, out);
    if (rc == MMHIP_OK) ctx->resident[key] = *out;
    return rc;
}

}  // namespace

extern "C" {

const char* mmhip_last_error(void) { return last_error_cstr(); }

const char* mmhip_version(void) { return "libmmhip 0.1 gfx950"; }

int mmhip_device_count(void) {
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess) return 0;
    return count;
}

int mmhip_is_available(void) { return gfx950_present(nullptr) ? 1 : 0; }

int mmhip_init(mmhip_ctx** out_ctx, int device) {
    if (!out_ctx) {
        set_error(MMHIP_ERR_INVALID, "init: null output pointer");
        return MMHIP_ERR_INVALID;
    }
    *out_ctx = nullptr;
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count == 0) {
        set_error(MMHIP_ERR_UNAVAILABLE, "init: no HIP device");
        return MMHIP_ERR_UNAVAILABLE;
    }
    if (device < 0 || device >= count) {
        set_error(MMHIP_ERR_INVALID, "init: device index out of range");
        return MMHIP_ERR_INVALID;
    }
    hipDeviceProp_t prop;
    hipError_t e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) return hip_fail(e, "init: hipGetDeviceProperties");
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        set_error(MMHIP_ERR_UNAVAILABLE, std::string("init: device is ") + prop.gcnArchName +
                                             ", this library is built for gfx950 only");
        return MMHIP_ERR_UNAVAILABLE;
    }
    e = hipSetDevice(device);
    if (e != hipSuccess) return hip_fail(e, "init: hipSetDevice");
    mmhip_ctx* ctx = new mmhip_ctx();
    ctx->device = device;
    ctx->num_cu = prop.multiProcessorCount;
    e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete ctx;
        return hip_fail(e, "init: hipStreamCreate");
    }
    // This device's address of the fixed scratch of mmhip_qmm_dev_noalloc,
    // looked up once per device with the device current.
    e = noalloc_scratch(device, &ctx->noalloc);
    if (e != hipSuccess) {
        (void)hipStreamDestroy(ctx->stream);
        delete ctx;
        return hip_fail(e, "init: scratch symbol address");
    }
    e = hipHostMalloc((void**)&ctx->status, sizeof(uint32_t), hipHostMallocDefault);
    if (e == hipSuccess) e = hipHostGetDevicePointer((void**)&ctx->status_dev, ctx->status, 0);
    if (e != hipSuccess) {
        if (ctx->status) (void)hipHostFree(ctx->status);
        (void)hipStreamDestroy(ctx->stream);
        delete ctx;
        return hip_fail(e, "init: status word");
    }
    *ctx->status = 0;
    *out_ctx = ctx;
    return MMHIP_OK;
}

void mmhip_destroy(mmhip_ctx* ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
    for (auto& kv : ctx->resident) weight_destroy(kv.second);
    ctx->resident.clear();
    ctx->d_in.release();
    ctx->d_out.release();
    ctx->d_raw.release();
    ctx->d_q.release();
    ctx->d_arg.release();
    ctx->h_in.release();
    ctx->h_out.release();
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    if (ctx->status) (void)hipHostFree(ctx->status);
    delete ctx;
}

int mmhip_synchronize(mmhip_ctx* ctx) {
    if (int rc = require_ctx(ctx)) return rc;
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return hip_fail(e, "synchronize");
    return check_device_status(ctx, "synchronize");
}

void* mmhip_stream(mmhip_ctx* ctx) { return ctx ? (void*)ctx->stream : nullptr; }

int mmhip_num_cu(mmhip_ctx* ctx) { return ctx ? ctx->num_cu : 0; }

int mmhip_profile_enable(mmhip_ctx* ctx, int enable) {
    if (int rc = require_ctx(ctx)) return rc;
    std::lock_guard<std::mutex> lk(ctx->mu);
    (void)hipStreamSynchronize(ctx->stream);
    ctx->timer.reset();
    ctx->timer.on = enable != 0;
    return MMHIP_OK;
}

int mmhip_profile_read(mmhip_ctx* ctx, const char* family, double* total_ms, uint64_t* launches) {
    if (int rc = require_ctx(ctx)) return rc;
    if (!family) {
        set_error(MMHIP_ERR_INVALID, "profile_read: null family");
        return MMHIP_ERR_INVALID;
    }
    std::lock_guard<std::mutex> lk(ctx->mu);
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return hip_fail(e, "profile_read");
    ctx->timer.drain();
    auto it = ctx->timer.totals.find(family);
    if (total_ms) *total_ms = it == ctx->timer.totals.end() ? 0.0 : it->second.first;
    if (launches) *launches = it == ctx->timer.totals.end() ? 0 : it->second.second;
    return MMHIP_OK;
}

int mmhip_malloc(mmhip_ctx* ctx, void** out_dev, size_t bytes) {
    if (int rc = require_ctx(ctx)) return rc;
    if (!out_dev) {
        set_error(MMHIP_ERR_INVALID, "malloc: null output pointer");
        return MMHIP_ERR_INVALID;
    }
    hipError_t e = hipMalloc(out_dev, bytes ? bytes : 1);
    if (e != hipSuccess) {
        *out_dev = nullptr;
        set_error(MMHIP_ERR_NOMEM, std::string("malloc: ") + hipGetErrorString(e));
        return MMHIP_ERR_NOMEM;
    }
    return MMHIP_OK;
}

int mmhip_free(mmhip_ctx* ctx, void* dev) {
    if (int rc = require_ctx(ctx)) return rc;
    if (!dev) return MMHIP_OK;
    hipError_t e = hipFree(dev);
    return e == hipSuccess ? MMHIP_OK : hip_fail(e, "free");
}

int mmhip_memcpy_h2d(mmhip_ctx* ctx, void* dst, const void* src, size_t bytes) {
    if (int rc = require_ctx(ctx)) return rc;
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    return e == hipSuccess ? MMHIP_OK : hip_fail(e, "memcpy_h2d");
}

int mmhip_memcpy_d2h(mmhip_ctx* ctx, void* dst, const void* src, size_t bytes) {
    if (int rc = require_ctx(ctx)) return rc;
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    return e == hipSuccess ? MMHIP_OK : hip_fail(e, "memcpy_d2h");
}

int mmhip_memset_dev(mmhip_ctx* ctx, void* dst, int value, size_t bytes) {
    if (int rc = require_ctx(ctx)) return rc;
    hipError_t e = hipMemsetAsync(dst, value, bytes, ctx->stream);
    return e == hipSuccess ? MMHIP_OK : hip_fail(e, "memset");
}

int mmhip_weight_upload(mmhip_ctx* ctx, const void* raw_host, uint32_t type, uint64_t rows, uint64_t cols,
                        uint64_t count, mmhip_weight** out_w) {
    if (int rc = require_ctx(ctx)) return rc;
    if (!raw_host || !out_w) {
        set_error(MMHIP_ERR_INVALID, "weight_upload: null pointer");
        return MMHIP_ERR_INVALID;
    }
    std::lock_guard<std::mutex> lk(ctx->mu);
    return weight_create(ctx, raw_host, false, type, rows, cols, count, out_w);
}

int mmhip_weight_from_device(mmhip_ctx* ctx, const void* raw_dev, uint32_t type, uint64_t rows, uint64_t cols,
                             uint64_t count, mmhip_weight** out_w) {
    if (int rc = require_ctx(ctx)) return rc;
    if (!raw_dev || !out_w) {
        set_error(MMHIP_ERR_INVALID, "weight_from_device: null pointer");
        return MMHIP_ERR_INVALID;
    }
    std::lock_guard<std::mutex> lk(ctx->mu);
    return weight_create(ctx, raw_dev, true, type, rows, cols, count, out_w);
}

void mmhip_weight_free(mmhip_ctx* ctx, mmhip_weight* w) {
    if (!w) return;
    if (ctx) (void)hipStreamSynchronize(ctx->stream);
    weight_destroy(w);
}

uint64_t mmhip_weight_device_bytes(const mmhip_weight* w) { return w ? w->bytes : 0; }

int mmhip_mat_vec_mul(mmhip_ctx* ctx, float* out, const void* ptr, uint32_t type, const float* x,
                      uint64_t out_dim, uint64_t in_dim) {
    return mmhip_batch_mat_mul(ctx, out, ptr, type, x, out_dim, 1, in_dim);
}

int mmhip_batch_mat_mul(mmhip_ctx* ctx, float* out, const void* ptr, uint32_t type, const float* in,
                        uint64_t out_dim, uint64_t batch, uint64_t in_dim) {
    if (int rc = require_ctx(ctx)) return rc;
    if (batch == 0 || out_dim == 0) return MMHIP_OK;
    if (!out || !ptr || !in || in_dim == 0) {
        set_error(MMHIP_ERR_INVALID, "mat_mul: null pointer or zero in_dim");
        return MMHIP_ERR_INVALID;
    }
    std::lock_guard<std::mutex> lk(ctx->mu);
    mmhip_weight* w = nullptr;
    int rc = resident_weight(ctx, ptr, type, out_dim, in_dim, &w);
    if (rc) return rc;
    const size_t in_bytes = batch * in_dim * 4, out_bytes = batch * out_dim * 4;
    hipError_t e = ctx->h_in.ensure(in_bytes);
    if (e == hipSuccess) e = ctx->h_out.ensure(out_bytes);
    if (e == hipSuccess) e = ctx->d_in.ensure(in_bytes);
    if (e == hipSuccess) e = ctx->d_out.ensure(out_bytes);
    if (e != hipSuccess) return hip_fail(e, "mat_mul: staging");
    std::memcpy(ctx->h_in.p, in, in_bytes);
    e = hipMemcpyAsync(ctx->d_in.p, ctx->h_in.p, in_bytes, hipMemcpyHostToDevice, ctx->stream);
    if (e != hipSuccess) return hip_fail(e, "mat_mul: H2D");
    const float* dx = static_cast<const float*>(ctx->d_in.p);
    float* dy = static_cast<float*>(ctx->d_out.p);
    if (batch == 1)
        rc = gemv_device(ctx, w, 0, 1, dx, 0, dy, 0, &ctx->d_q);
    else
        rc = qmm_device(ctx, w, 0, dx, dy, batch, 0, &ctx->d_q);
    if (rc) return rc;
    e = hipMemcpyAsync(ctx->h_out.p, dy, out_bytes, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return hip_fail(e, "mat_mul: D2H");
    std::memcpy(out, ctx->h_out.p, out_bytes);
    return MMHIP_OK;
}

int mmhip_dequantize(mmhip_ctx* ctx, float* out, const void* data, uint32_t type, uint64_t n) {
    if (int rc = require_ctx(ctx)) return rc;
    if (n == 0) return MMHIP_OK;
    if (!out || !data) {
        set_error(MMHIP_ERR_INVALID, "dequantize: null pointer");
        return MMHIP_ERR_INVALID;
    }
    const uint64_t raw_bytes = tensor_bytes(type, n);
    if (raw_bytes == 0) {
        set_error(MMHIP_ERR_UNSUPPORTED, "dequantize: unsupported GgmlType " + std::to_string(type));
        return MMHIP_ERR_UNSUPPORTED;
    }
    std::lock_guard<std::mutex> lk(ctx->mu);
    hipError_t e = ctx->d_raw.ensure(raw_bytes);
    if (e == hipSuccess) e = ctx->d_out.ensure(n * 4);
    if (e != hipSuccess) return hip_fail(e, "dequantize: scratch");
    e = hipMemcpyAsync(ctx->d_raw.p, data, raw_bytes, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = launch_dequant(ctx->d_raw.p, type, n, static_cast<float*>(ctx->d_out.p), ctx->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(out, ctx->d_out.p, n * 4, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    return e == hipSuccess ? MMHIP_OK : hip_fail(e, "dequantize");
}

int mmhip_forget(mmhip_ctx* ctx, const void* ptr) {
    if (int rc = require_ctx(ctx)) return rc;
    std::lock_guard<std::mutex> lk(ctx->mu);
    (void)hipStreamSynchronize(ctx->stream);
    for (auto it = ctx->resident.begin(); it != ctx->resident.end();) {
        if (std::get<0>(it->first) == ptr) {
            weight_destroy(it->second);
            it = ctx->resident.erase(it);
        } else {
            ++it;
        }
    }
    return MMHIP_OK;
}

int mmhip_dequantize_dev(mmhip_ctx* ctx, float* out_dev, const void* raw_dev, uint32_t type, uint64_t n) {
    if (int rc = require_ctx(ctx)) return rc;
    if (tensor_bytes(type, 1) == 0) {
        set_error(MMHIP_ERR_UNSUPPORTED, "dequantize_dev: unsupported GgmlType " + std::to_string(type));
        return MMHIP_ERR_UNSUPPORTED;
    }
    hipError_t e = launch_dequant(raw_dev, type, n, out_dev, ctx->stream);
    return e == hipSuccess ? MMHIP_OK : hip_fail(e, "dequantize_dev");
}

int mmhip_quantize_q8_0_rows_dev(mmhip_ctx* ctx, void* blocks_dev, const float* x_dev, uint64_t x_stride,
                                 uint64_t n_rows, uint32_t row_len) {
    if (int rc = require_ctx(ctx)) return rc;
    if (n_rows == 0 || row_len == 0) return MMHIP_OK;
    if (!blocks_dev || !x_dev || x_stride < row_len) {
        set_error(MMHIP_ERR_INVALID, "quantize_q8_0_rows_dev: null pointer or x_stride < row_len");
        return MMHIP_ERR_INVALID;
    }
    if (reinterpret_cast<uintptr_t>(blocks_dev) & 3u) {
        set_error(MMHIP_ERR_INVALID, "quantize_q8_0_rows_dev: blocks_dev must be 4-byte aligned");
        return MMHIP_ERR_INVALID;
    }
    hipError_t e = launch_quantize_q8_0_rows(x_dev, x_stride, n_rows, row_len, blocks_dev, ctx->stream);
    return e == hipSuccess ? MMHIP_OK : hip_fail(e, "quantize_q8_0_rows_dev");
}

int mmhip_dequantize_q8_0_rows_dev(mmhip_ctx* ctx, float* out_dev, uint64_t out_stride, const void* blocks_dev,
                                   uint64_t n_rows, uint32_t row_len) {
    if (int rc = require_ctx(ctx)) return rc;
    if (n_rows == 0 || row_len == 0) return MMHIP_OK;
    if (!blocks_dev || !out_dev || out_stride < row_len) {
        set_error(MMHIP_ERR_INVALID, "dequantize_q8_0_rows_dev: null pointer or out_stride < row_len");
        return MMHIP_ERR_INVALID;
    }
    if (reinterpret_cast<uintptr_t>(blocks_dev) & 1u) {
        set_error(MMHIP_ERR_INVALID, "dequantize_q8_0_rows_dev: blocks_dev must be 2-byte aligned");
        return MMHIP_ERR_INVALID;
    }
    hipError_t e = launch_dequantize_q8_0_rows(blocks_dev, n_rows, row_len, out_dev, out_stride, ctx->stream);
    return e == hipSuccess ? MMHIP_OK : hip_fail(e, "dequantize_q8_0_rows_dev");
}

int mmhip_quantize_q8_0(mmhip_ctx* ctx, void* blocks_host, const float* x_host, uint64_t n) {
    if (int rc = require_ctx(ctx)) return rc;
    if (n == 0) return MMHIP_OK;
    if (!blocks_host || !x_host) {
        set_error(MMHIP_ERR_INVALID, "quantize_q8_0: null pointer");
        return MMHIP_ERR_INVALID;
    }
    const uint64_t out_bytes = (n + 31) / 32 * 34;
    std::lock_guard<std::mutex> lk(ctx->mu);
    hipError_t e = ctx->d_out.ensure(n * 4);
    if (e == hipSuccess) e = ctx->d_raw.ensure(out_bytes);
    if (e != hipSuccess) return hip_fail(e, "quantize_q8_0: scratch");
    e = hipMemcpyAsync(ctx->d_out.p, x_host, n * 4, hipMemcpyHostToDevice, ctx->stream);
    // One row of n values: the blocks of quantizeQ8_0 over the whole array.
    if (e == hipSuccess) {
        if (n > 0xFFFFFFFFull) e = hipErrorInvalidValue;
        else e = launch_quantize_q8_0_rows(static_cast<const float*>(ctx->d_out.p), n, 1, (uint32_t)n, ctx->d_raw.p,
                                           ctx->stream);
    }
    if (e == hipSuccess) e = hipMemcpyAsync(blocks_host, ctx->d_raw.p, out_bytes, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    return e == hipSuccess ? MMHIP_OK : hip_fail(e, "quantize_q8_0");
}

int mmhip_argmax_dev(mmhip_ctx* ctx, uint32_t* out_dev, const float* logits_dev, uint64_t n) {
    if (int rc = require_ctx(ctx)) return rc;
    if (!out_dev || !logits_dev || n == 0 || n > 0xFFFFFFFFull) {
        set_error(MMHIP_ERR_INVALID, "argmax_dev: null pointer or n outside [1, 2^32)");
        return MMHIP_ERR_INVALID;
    }
    std::lock_guard<std::mutex> lk(ctx->mu);
    hipError_t e = ctx->d_arg.ensure(argmax_scratch_bytes(n));
    if (e == hipSuccess) e = launch_argmax(logits_dev, n, out_dev, ctx->d_arg.p, ctx->stream);
    return e == hipSuccess ? MMHIP_OK : hip_fail(e, "argmax_dev");
}

int mmhip_sample_greedy(mmhip_ctx* ctx, uint32_t* out_host, const float* logits_host, uint64_t n) {
    if (int rc = require_ctx(ctx)) return rc;
    if (!out_host || !logits_host || n == 0 || n > 0xFFFFFFFFull) {
        set_error(MMHIP_ERR_INVALID, "sample_greedy: null pointer or n outside [1, 2^32)");
        return MMHIP_ERR_INVALID;
    }
    std::lock_guard<std::mutex> lk(ctx->mu);
    hipError_t e = ctx->d_out.ensure(n * 4);
    if (e == hipSuccess) e = ctx->d_raw.ensure(4);
    if (e == hipSuccess) e = ctx->d_arg.ensure(argmax_scratch_bytes(n));
    if (e != hipSuccess) return hip_fail(e, "sample_greedy: scratch");
    e = hipMemcpyAsync(ctx->d_out.p, logits_host, n * 4, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess)
        e = launch_argmax(static_cast<const float*>(ctx->d_out.p), n, static_cast<uint32_t*>(ctx->d_raw.p),
                          ctx->d_arg.p, ctx->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(out_host, ctx->d_raw.p, 4, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    return e == hipSuccess ? MMHIP_OK : hip_fail(e, "sample_greedy");
}

int mmhip_gemv_dev(mmhip_ctx* ctx, const mmhip_weight* w, uint64_t mat, const float* x_dev, float* y_dev) {
    return mmhip_gemv_batched_dev(ctx, w, mat, 1, x_dev, 0, y_dev, 0);
}

int mmhip_gemv_batched_dev(mmhip_ctx* ctx, const mmhip_weight* w, uint64_t first, uint64_t n_mats,
                           const float* x_dev, uint64_t x_stride, float* y_dev, uint64_t y_stride) {
    if (int rc = require_ctx(ctx)) return rc;
    if (!w || !x_dev || !y_dev) {
        set_error(MMHIP_ERR_INVALID, "gemv_dev: null pointer");
        return MMHIP_ERR_INVALID;
    }
    std::lock_guard<std::mutex> lk(ctx->mu);
    return gemv_device(ctx, w, first, n_mats, x_dev, x_stride, y_dev, y_stride, &ctx->d_q);
}

int mmhip_gemv_grouped_dev(mmhip_ctx* ctx, const mmhip_gemv_group* groups, uint32_t n_groups) {
    if (int rc = require_ctx(ctx)) return rc;
    if (!groups || n_groups == 0 || n_groups > MMHIP_GEMV_MAX_GROUPS) {
        set_error(MMHIP_ERR_INVALID, "gemv_grouped_dev: need 1.." + std::to_string(MMHIP_GEMV_MAX_GROUPS) + " groups");
        return MMHIP_ERR_INVALID;
    }
    GemvArgs segs[MMHIP_GEMV_MAX_GROUPS];
    uint32_t fmt = 0;
    for (uint32_t i = 0; i < n_groups; ++i) {
        const mmhip_gemv_group& gr = groups[i];
        if (!gr.w || !gr.x_dev || !gr.y_dev) {
            set_error(MMHIP_ERR_INVALID, "gemv_grouped_dev: null pointer in group " + std::to_string(i));
            return MMHIP_ERR_INVALID;
        }
        if (gr.w->type == kF32 || gr.w->type == kF16) {
            set_error(MMHIP_ERR_UNSUPPORTED, "gemv_grouped_dev: quantised weights only (Q8_0, IQ2_XXS)");
            return MMHIP_ERR_UNSUPPORTED;
        }
        if (gr.first + gr.n_mats > gr.w->count || gr.first + gr.n_mats < gr.first) {
            set_error(MMHIP_ERR_INVALID, "gemv_grouped_dev: matrix range out of the weight in group " + std::to_string(i));
            return MMHIP_ERR_INVALID;
        }
        if (i > 0 && gr.w->geom.fmt != fmt) {
            set_error(MMHIP_ERR_INVALID, "gemv_grouped_dev: all groups must share one weight type");
            return MMHIP_ERR_INVALID;
        }
        fmt = gr.w->geom.fmt;
        segs[i] = gemv_args(gr.w, gr.first, gr.n_mats, gr.x_dev, gr.x_stride, gr.y_dev, gr.y_stride);
    }
    std::lock_guard<std::mutex> lk(ctx->mu);
    hipError_t e;
    {
        TimedLaunch tl(ctx, "gemv_q");
        e = launch_gemv_segments(segs, n_groups, fmt, ctx->num_cu, ctx->stream);
    }
    return e == hipSuccess ? MMHIP_OK : hip_fail(e, "gemv_grouped_dev: launch");
}

int mmhip_qmm_dev(mmhip_ctx* ctx, const mmhip_weight* w, uint64_t mat, const float* x_dev, float* y_dev,
                  uint64_t batch, int out_layout) {
    if (int rc = require_ctx(ctx)) return rc;
    if (!w || !x_dev || !y_dev || (out_layout != 0 && out_layout != 1)) {
        set_error(MMHIP_ERR_INVALID, "qmm_dev: null pointer or bad layout");
        return MMHIP_ERR_INVALID;
    }
    std::lock_guard<std::mutex> lk(ctx->mu);
    return qmm_device(ctx, w, mat, x_dev, y_dev, batch, out_layout, &ctx->d_q);
}

int mmhip_qmm_dev_noalloc(mmhip_ctx* ctx, const mmhip_weight* w, uint64_t mat, const float* x_dev, float* y_dev,
                          uint64_t batch, int out_layout) {
    if (int rc = require_ctx(ctx)) return rc;
    if (!w || !x_dev || !y_dev || (out_layout != 0 && out_layout != 1)) {
        set_error(MMHIP_ERR_INVALID, "qmm_dev_noalloc: null pointer or bad layout");
        return MMHIP_ERR_INVALID;
    }
    if (batch == 0) return MMHIP_OK;
    if (mat >= w->count) {
        set_error(MMHIP_ERR_INVALID, "qmm_dev_noalloc: matrix index out of range");
        return MMHIP_ERR_INVALID;
    }
    if (w->type == kF32 || w->type == kF16) {
        // No scratch on this branch: the same launch as mmhip_qmm_dev.
        std::lock_guard<std::mutex> lk(ctx->mu);
        return qmm_device(ctx, w, mat, x_dev, y_dev, batch, out_layout, nullptr);
    }
    const size_t need = quant_act_bytes(batch, w->geom.cols_pad);
    if (need > MMHIP_NOALLOC_SCRATCH_BYTES) {
        set_error(MMHIP_ERR_INVALID, "qmm_dev_noalloc: batch " + std::to_string(batch) + " x " +
                                         std::to_string(w->geom.cols_pad) + " padded columns needs " +
                                         std::to_string(need) + " bytes of scratch, above the fixed " +
                                         std::to_string(MMHIP_NOALLOC_SCRATCH_BYTES));
        return MMHIP_ERR_INVALID;
    }
    if (!ctx->noalloc) {
        set_error(MMHIP_ERR_HIP, "qmm_dev_noalloc: no scratch address for this device");
        return MMHIP_ERR_HIP;
    }
    std::lock_guard<std::mutex> lk(ctx->mu);
    return qmm_quantised(ctx, w, mat, x_dev, y_dev, batch, out_layout, ctx->noalloc, false);
}

}  // extern "C"
