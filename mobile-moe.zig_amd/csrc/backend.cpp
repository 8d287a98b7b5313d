// HipBackend internals: error state, scratch buffers, weight upload + repack,
// and the device-pointer GEMV / QMM drivers used by every entry point.
#include "backend.hpp"

#include <cstdlib>
#include <cstring>
#include <string>

#include "../../include/mmhip.h"

namespace mmhip {

namespace {
thread_local std::string t_err;
}  // namespace

const char* last_error_cstr() { return t_err.c_str(); }

void set_error(int code, const std::string& msg) {
    (void)code;
    t_err = msg;
}

int hip_fail(hipError_t e, const char* what) {
    set_error(MMHIP_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
    return MMHIP_ERR_HIP;
}

int check_device_status(mmhip_ctx* ctx, const char* what) {
    const uint32_t st = ctx->status ? __atomic_load_n(ctx->status, __ATOMIC_ACQUIRE) : 0u;
    if (st == 0) return MMHIP_OK;
    __atomic_store_n(ctx->status, 0u, __ATOMIC_RELEASE);
    set_error(MMHIP_ERR_HIP, std::string(what) + ": decode MoE launch: a grid-wide wait timed out (code " +
                                 std::to_string(st) + "); its output is invalid");
    return MMHIP_ERR_HIP;
}

uint64_t block_size(uint32_t type) {
    switch (type) {
        case kF32: case kF16: return 1;
        case kQ8_0: return 32;
        case kIq2Xxs: return 256;
        default: return 0;
    }
}

uint64_t block_bytes(uint32_t type) {
    switch (type) {
        case kF32: return 4;
        case kF16: return 2;
        case kQ8_0: return 34;
        case kIq2Xxs: return 66;
        default: return 0;
    }
}

uint64_t tensor_bytes(uint32_t type, uint64_t n) {
    const uint64_t bs = block_size(type);
    if (bs == 0) return 0;
    return ((n + bs - 1) / bs) * block_bytes(type);
}

hipError_t DevBuf::ensure(size_t bytes) {
    if (bytes <= cap) return hipSuccess;
    release();
    size_t want = bytes < 4096 ? 4096 : bytes;
    hipError_t e = hipMalloc(&p, want);
    if (e != hipSuccess) {
        p = nullptr;
        return e;
    }
    cap = want;
    return hipSuccess;
}

void DevBuf::release() {
    if (p) (void)hipFree(p);
    p = nullptr;
    cap = 0;
}

hipError_t HostBuf::ensure(size_t bytes) {
    if (bytes <= cap) return hipSuccess;
    release();
    size_t want = bytes < 4096 ? 4096 : bytes;
    hipError_t e = hipHostMalloc(&p, want, hipHostMallocDefault);
    if (e != hipSuccess) {
        p = nullptr;
        return e;
    }
    cap = want;
    return hipSuccess;
}

void HostBuf::release() {
    if (p) (void)hipHostFree(p);
    p = nullptr;
    cap = 0;
}

static uint64_t round_up(uint64_t v, uint64_t m) { return (v + m - 1) / m * m; }

QuantAct quant_act_view(void* base, uint64_t n_vec, uint64_t cols_pad) {
    const uint64_t stride = round_up(cols_pad, 64);
    QuantAct q;
    q.hi = static_cast<int8_t*>(base);
    q.lo = q.hi + n_vec * stride;
    q.scale = reinterpret_cast<float*>(q.lo + n_vec * stride);
    q.stride = stride;
    q.scale_stride = stride / 32;
    return q;
}

size_t quant_act_bytes(uint64_t n_vec, uint64_t cols_pad) {
    const uint64_t stride = round_up(cols_pad, 64);
    return (size_t)(2 * n_vec * stride + n_vec * (stride / 32) * 4);
}

int weight_create(mmhip_ctx* ctx, const void* raw, bool raw_on_device, uint32_t type, uint64_t rows,
                  uint64_t cols, uint64_t count, mmhip_weight** out) {
    const WeightSegment seg{raw, count};
    return weight_create_segments(ctx, &seg, 1, raw_on_device, type, rows, cols, out);
}

int weight_create_segments(mmhip_ctx* ctx, const WeightSegment* segs, size_t n_segs, bool raw_on_device,
                           uint32_t type, uint64_t rows, uint64_t cols, mmhip_weight** out) {
    *out = nullptr;
    uint64_t count = 0;
    for (size_t i = 0; i < n_segs; ++i) {
        if (!segs[i].raw && segs[i].count) {
            set_error(MMHIP_ERR_INVALID, "weight: null source");
            return MMHIP_ERR_INVALID;
        }
        count += segs[i].count;
    }
    if (rows == 0 || cols == 0 || count == 0) {
        set_error(MMHIP_ERR_INVALID, "weight: rows, cols and count must be > 0");
        return MMHIP_ERR_INVALID;
    }
    if (block_size(type) == 0) {
        set_error(MMHIP_ERR_UNSUPPORTED, "weight: GgmlType " + std::to_string(type) +
                                             " is not on this backend's path (F32, F16, Q8_0, IQ2_XXS)");
        return MMHIP_ERR_UNSUPPORTED;
    }
    if (type == kIq2Xxs && cols % 256 != 0) {
        set_error(MMHIP_ERR_INVALID, "weight: IQ2_XXS rows must hold whole 256-element superblocks");
        return MMHIP_ERR_INVALID;
    }
    const uint64_t row_bytes = ((cols + block_size(type) - 1) / block_size(type)) * block_bytes(type);
    const uint64_t mat_bytes = row_bytes * rows;
    const uint64_t raw_bytes = mat_bytes * count;
    // Copies every segment to dst (device) back to back.
    auto gather = [&](char* dst) -> hipError_t {
        uint64_t off = 0;
        for (size_t i = 0; i < n_segs; ++i) {
            const uint64_t b = segs[i].count * mat_bytes;
            if (!b) continue;
            hipError_t e = hipMemcpyAsync(dst + off, segs[i].raw, b,
                                          raw_on_device ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice,
                                          ctx->stream);
            if (e != hipSuccess) return e;
            off += b;
        }
        return hipSuccess;
    };
    mmhip_weight* w = new mmhip_weight();
    w->type = type;
    w->rows = rows;
    w->cols = cols;
    w->count = count;
    hipError_t e;
    if (type == kF32 || type == kF16) {
        e = hipMalloc(&w->plain, raw_bytes);
        if (e != hipSuccess) {
            delete w;
            return hip_fail(e, "weight: hipMalloc");
        }
        w->bytes = raw_bytes;
        e = gather(static_cast<char*>(w->plain));
        if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) {
            weight_destroy(w);
            return hip_fail(e, "weight: upload");
        }
        *out = w;
        return MMHIP_OK;
    }
    TileGeom& g = w->geom;
    g.fmt = (type == kIq2Xxs) ? kFmtIq2 : kFmtQ8;
    g.rows = rows;
    g.cols = cols;
    g.count = count;
    g.tiles = (rows + 15) / 16;
    g.unit_cols = (type == kIq2Xxs) ? 256 : 64;
    // Q8_0 tiles hold whole 256-column activation groups (zero units pad).
    g.units = (type == kIq2Xxs) ? cols / 256 : ((((cols + 31) / 32 + 1) / 2 + 3) / 4) * 4;
    g.cols_pad = g.units * g.unit_cols;
    g.rec_stride = g.tiles * g.units * 64;
    // Scales are stored per row ([tile][row][unit]) so that one vector load
    // fetches a row's scales for several units.
    g.d_row = ((g.units * ((type == kIq2Xxs) ? 1 : 2) + 7) / 8) * 8;
    g.d_stride = g.tiles * 16 * g.d_row;
    // Every kernel reads one matrix through a buffer resource with 32-bit
    // offsets, 2^31 being its out-of-range sentinel.
    if (g.rec_stride * 16 >= 0x80000000ull || g.d_stride * 2 >= 0x80000000ull) {
        delete w;
        set_error(MMHIP_ERR_UNSUPPORTED, "weight: one repacked matrix must stay below 2 GiB");
        return MMHIP_ERR_UNSUPPORTED;
    }
    const size_t rec_bytes = (size_t)(g.rec_stride * count * 16);
    const size_t d_bytes = (size_t)(g.d_stride * count * 2);
    e = hipMalloc(&w->recs, rec_bytes);
    if (e == hipSuccess) e = hipMalloc(&w->dvals, d_bytes);
    if (e != hipSuccess) {
        weight_destroy(w);
        return hip_fail(e, "weight: hipMalloc");
    }
    w->bytes = rec_bytes + d_bytes;
    e = hipMemsetAsync(w->dvals, 0, d_bytes, ctx->stream);  // row padding stays zero
    if (e != hipSuccess) {
        weight_destroy(w);
        return hip_fail(e, "weight: memset");
    }
    const void* src = segs[0].raw;
    if (!raw_on_device || n_segs > 1) {
        e = ctx->d_raw.ensure(raw_bytes);
        if (e == hipSuccess) e = gather(static_cast<char*>(ctx->d_raw.p));
        if (e != hipSuccess) {
            weight_destroy(w);
            return hip_fail(e, "weight: upload");
        }
        src = ctx->d_raw.p;
    }
    e = launch_repack(src, g, w->recs, w->dvals, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        weight_destroy(w);
        return hip_fail(e, "weight: repack");
    }
    *out = w;
    return MMHIP_OK;
}

void weight_destroy(mmhip_weight* w) {
    if (!w) return;
    if (w->recs) (void)hipFree(w->recs);
    if (w->dvals) (void)hipFree(w->dvals);
    if (w->plain) (void)hipFree(w->plain);
    delete w;
}

int gemv_device(mmhip_ctx* ctx, const mmhip_weight* w, uint64_t first, uint64_t n, const float* x,
                uint64_t x_stride, float* y, uint64_t y_stride, DevBuf* qscratch) {
    if (n == 0) return MMHIP_OK;
    if (first + n > w->count) {
        set_error(MMHIP_ERR_INVALID, "gemv: matrix index out of range");
        return MMHIP_ERR_INVALID;
    }
    hipError_t e;
    if (w->type == kF32 || w->type == kF16) {
        const uint64_t es = (w->type == kF32) ? 4 : 2;
        const uint64_t mstride = w->rows * w->cols;
        const char* base = static_cast<const char*>(w->plain) + first * mstride * es;
        {
            TimedLaunch tl(ctx, "gemv_float");
            e = launch_gemv_float(base, w->type, mstride, x, x_stride, y, y_stride, (uint32_t)n, (uint32_t)w->rows,
                                  (uint32_t)w->cols, ctx->stream);
        }
        return e == hipSuccess ? MMHIP_OK : hip_fail(e, "gemv: launch");
    }
    (void)qscratch;
    const GemvArgs a = gemv_args(w, first, n, x, x_stride, y, y_stride);
    {
        TimedLaunch tl(ctx, "gemv_q");
        e = launch_gemv_q(a, w->geom.fmt, ctx->num_cu, ctx->stream);
    }
    return e == hipSuccess ? MMHIP_OK : hip_fail(e, "gemv: launch");
}

GemvArgs gemv_args(const mmhip_weight* w, uint64_t first, uint64_t n, const float* x, uint64_t x_stride, float* y,
                   uint64_t y_stride) {
    const TileGeom& g = w->geom;
    GemvArgs a{};
    a.recs = w->recs;
    a.dvals = w->dvals;
    a.rec_stride = g.rec_stride;
    a.d_stride = g.d_stride;
    a.d_row = (uint32_t)g.d_row;
    a.x = x;
    a.x_stride = x_stride;
    a.y = y;
    a.y_stride = y_stride;
    a.probs = nullptr;
    a.n_active = nullptr;
    a.x2_off = 0;
    a.silu_mul = 0;
    a.first_mat = first;
    a.n_probs = (uint32_t)n;
    a.tiles = (uint32_t)g.tiles;
    a.units = (uint32_t)g.units;
    a.rows = (uint32_t)g.rows;
    a.cols = (uint32_t)g.cols;
    a.tiles_per_wg = 0;
    return a;
}

int qmm_device(mmhip_ctx* ctx, const mmhip_weight* w, uint64_t mat, const float* x, float* y, uint64_t batch,
               int out_layout, DevBuf* qscratch) {
    if (batch == 0) return MMHIP_OK;
    if (mat >= w->count) {
        set_error(MMHIP_ERR_INVALID, "qmm: matrix index out of range");
        return MMHIP_ERR_INVALID;
    }
    hipError_t e;
    if (w->type == kF32 || w->type == kF16) {
        if (out_layout != 0) {
            set_error(MMHIP_ERR_UNSUPPORTED, "qmm: float weights support out_layout 0 only");
            return MMHIP_ERR_UNSUPPORTED;
        }
        const uint64_t es = (w->type == kF32) ? 4 : 2;
        const char* base = static_cast<const char*>(w->plain) + mat * w->rows * w->cols * es;
        e = launch_gemv_float(base, w->type, 0, x, w->cols, y, w->rows, (uint32_t)batch, (uint32_t)w->rows,
                              (uint32_t)w->cols, ctx->stream);
        return e == hipSuccess ? MMHIP_OK : hip_fail(e, "qmm: launch");
    }
    if (!qmm_fused(w, batch)) {
        e = qscratch->ensure(quant_act_bytes(batch, w->geom.cols_pad));
        if (e != hipSuccess) return hip_fail(e, "qmm: scratch");
    }
    return qmm_quantised(ctx, w, mat, x, y, batch, out_layout, qscratch->p, true);
}

bool qmm_fused(const mmhip_weight* w, uint64_t batch) {
    // MMHIP_QMM_FUSED=0: the two-launch path (quantize_kernel, then
    // group_kernel) for every shape.
    static const bool on = [] {
        const char* e = getenv("MMHIP_QMM_FUSED");
        return !(e && e[0] == '0');
    }();
    // The fused kernel addresses x (batch rows of cols floats) with 32-bit
    // byte offsets.
    return on && qmm_q8_fused_fits(w->geom) && batch * w->cols * 4 < 0x80000000ull;
}

int qmm_quantised(mmhip_ctx* ctx, const mmhip_weight* w, uint64_t mat, const float* x, float* y, uint64_t batch,
                  int out_layout, void* qbuf, bool timed) {
    const TileGeom& g = w->geom;
    const uint64_t ld = out_layout == 0 ? w->rows : batch;
    hipError_t e;
    if (qmm_fused(w, batch)) {
        // One launch, the activations quantised inside (qbuf unused).
        TimedLaunch tl(timed ? ctx : nullptr, "qmm");
        e = launch_qmm_q8_fused(w->recs, w->dvals, g, mat, x, w->cols, (uint32_t)w->cols, (uint32_t)batch, y, ld,
                                out_layout, ctx->stream);
        return e == hipSuccess ? MMHIP_OK : hip_fail(e, "qmm: launch");
    }
    // The quantiser writes every digit and scale of the batch x cols_pad
    // block it reads back (columns past cols as zeros), so qbuf needs no
    // clearing and keeps nothing from an earlier call.
    const QuantAct q = quant_act_view(qbuf, batch, g.cols_pad);
    {
        TimedLaunch tl(timed ? ctx : nullptr, "quantize");
        e = launch_quantize(x, w->cols, (uint32_t)batch, (uint32_t)w->cols, (uint32_t)g.cols_pad, q, ctx->stream,
                            g.fmt == kFmtIq2);
    }
    if (e != hipSuccess) return hip_fail(e, "qmm: quantize");
    {
        TimedLaunch tl(timed ? ctx : nullptr, "qmm");
        e = launch_group_dense(w->recs, w->dvals, g, mat, q, (uint32_t)batch, y, ld, out_layout, ctx->num_cu,
                               ctx->stream);
    }
    return e == hipSuccess ? MMHIP_OK : hip_fail(e, "qmm: launch");
}

}  // namespace mmhip

hipEvent_t KernelTimer::get() {
    if (!pool.empty()) {
        hipEvent_t e = pool.back();
        pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) return nullptr;
    return e;
}

void KernelTimer::begin(hipStream_t s, const char* family, hipEvent_t* a) {
    (void)family;
    *a = get();
    if (*a && hipEventRecord(*a, s) != hipSuccess) {
        pool.push_back(*a);
        *a = nullptr;
    }
}

void KernelTimer::end(hipStream_t s, const char* family, hipEvent_t a) {
    hipEvent_t b = get();
    if (!b) {
        pool.push_back(a);
        return;
    }
    if (hipEventRecord(b, s) != hipSuccess) {
        pool.push_back(a);
        pool.push_back(b);
        return;
    }
    pending.push_back(Rec{family, a, b});
}

void KernelTimer::drain() {
    for (auto& r : pending) {
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, r.a, r.b) == hipSuccess) {
            auto& t = totals[r.family];
            t.first += ms;
            t.second += 1;
        }
        pool.push_back(r.a);
        pool.push_back(r.b);
    }
    pending.clear();
}

void KernelTimer::reset() {
    for (auto& r : pending) {
        pool.push_back(r.a);
        pool.push_back(r.b);
    }
    pending.clear();
    totals.clear();
}

KernelTimer::~KernelTimer() {
    reset();
    for (hipEvent_t e : pool) (void)hipEventDestroy(e);
}
