// HipBackend: the C++ object behind the C ABI. It plays the role of the
// reference's OpenCLBackend (src/opencl_backend.zig:55-537): one device
// context, a residency cache of uploaded weights keyed by the host pointer
// (getOrUploadMatBuffer, 311-323), and the op entry points of the engine seam.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <map>
#include <mutex>
#include <string>
#include <tuple>
#include <vector>

#include "kernels/kernels.hpp"

namespace mmhip {

enum GgmlType : uint32_t { kF32 = 0, kF16 = 1, kQ8_0 = 8, kIq2Xxs = 16 };

// GgmlType.blockSize / blockBytes / tensorBytes (src/gguf.zig:59-117) for the
// types this backend accepts; 0 for the others.
uint64_t block_size(uint32_t type);
uint64_t block_bytes(uint32_t type);
uint64_t tensor_bytes(uint32_t type, uint64_t n_elements);

void set_error(int code, const std::string& msg);
int hip_fail(hipError_t e, const char* what);

// Growable device / pinned-host scratch buffer.
struct DevBuf {
    void* p = nullptr;
    size_t cap = 0;
    hipError_t ensure(size_t bytes);
    void release();
};
struct HostBuf {
    void* p = nullptr;
    size_t cap = 0;
    hipError_t ensure(size_t bytes);
    void release();
};

}  // namespace mmhip

// A device-resident stacked weight ([count][rows][cols]).
struct mmhip_weight {
    uint32_t type = 0;
    uint64_t rows = 0, cols = 0, count = 0;
    // Quantised types: tile layout.
    mmhip::TileGeom geom{};
    uint4* recs = nullptr;
    uint16_t* dvals = nullptr;
    // F32 / F16: row-major copy.
    void* plain = nullptr;
    uint64_t bytes = 0;
};

// Opt-in per-family kernel timing with HIP events (mmhip_profile_*).
struct KernelTimer {
    bool on = false;
    struct Rec { std::string family; hipEvent_t a, b; };
    std::vector<Rec> pending;
    std::map<std::string, std::pair<double, uint64_t>> totals;
    std::vector<hipEvent_t> pool;
    hipEvent_t get();
    void begin(hipStream_t s, const char* family, hipEvent_t* a);
    void end(hipStream_t s, const char* family, hipEvent_t a);
    void drain();   // requires the stream to be idle
    void reset();
    ~KernelTimer();
};

struct mmhip_ctx {
    int device = 0;
    int num_cu = 0;
    hipStream_t stream = nullptr;
    std::mutex mu;                   // seam calls: scratch + residency map
    std::map<std::tuple<const void*, uint32_t, uint64_t, uint64_t>, mmhip_weight*> resident;
    mmhip::DevBuf d_in, d_out, d_raw, d_q;
    mmhip::DevBuf d_arg;  // argmax partials (value, index) of the first pass
    mmhip::HostBuf h_in, h_out;
    void* noalloc = nullptr;  // this device's fixed QMM scratch (mmhip_qmm_dev_noalloc)
    // Pinned host word that device code sets when a grid-wide wait of the
    // one-launch decode MoE layer timed out (0: none); read after a sync.
    uint32_t* status = nullptr;
    uint32_t* status_dev = nullptr;
    KernelTimer timer;
};

// Brackets one kernel launch with timing events when profiling is on.
struct TimedLaunch {
    mmhip_ctx* ctx;
    const char* family;
    hipEvent_t a = nullptr;
    // A null ctx times nothing (callers that must not create events).
    TimedLaunch(mmhip_ctx* c, const char* f) : ctx(c), family(f) {
        if (ctx && ctx->timer.on) ctx->timer.begin(ctx->stream, family, &a);
    }
    ~TimedLaunch() {
        if (ctx && ctx->timer.on && a) ctx->timer.end(ctx->stream, family, a);
    }
};

namespace mmhip {

// MMHIP_OK, or MMHIP_ERR_HIP with a message when device code recorded a
// failure in the context's status word since the last check (which clears
// it). Call after the context's stream has been synchronised.
int check_device_status(mmhip_ctx* ctx, const char* what);

// Upload helpers shared by the ABI and the MoE layer.
int weight_create(mmhip_ctx* ctx, const void* raw, bool raw_on_device, uint32_t type, uint64_t rows,
                  uint64_t cols, uint64_t count, mmhip_weight** out);
// One stacked weight from several sources of `count` matrices each, in order.
struct WeightSegment {
    const void* raw;
    uint64_t count;
};
int weight_create_segments(mmhip_ctx* ctx, const WeightSegment* segs, size_t n_segs, bool raw_on_device,
                           uint32_t type, uint64_t rows, uint64_t cols, mmhip_weight** out);
void weight_destroy(mmhip_weight* w);

// Layout of quantised activations inside one scratch allocation.
QuantAct quant_act_view(void* base, uint64_t n_vec, uint64_t cols_pad);
size_t quant_act_bytes(uint64_t n_vec, uint64_t cols_pad);

// y_i = W[first + i] . x_i for i < n (device pointers, async). Quantised types
// quantise x into `qscratch` first.
int gemv_device(mmhip_ctx* ctx, const mmhip_weight* w, uint64_t first, uint64_t n, const float* x,
                uint64_t x_stride, float* y, uint64_t y_stride, DevBuf* qscratch);
// The quantised branch of qmm_device with the activation digits in `qbuf`
// (at least quant_act_bytes(batch, cols_pad) bytes; unused where qmm_fused
// holds); allocates nothing, and records timing events only when `timed`.
int qmm_quantised(mmhip_ctx* ctx, const mmhip_weight* w, uint64_t mat, const float* x, float* y, uint64_t batch,
                  int out_layout, void* qbuf, bool timed);
// Kernel arguments of a GEMV over matrices [first, first + n) of a quantised
// weight (x_i = x + i * x_stride, y_i = y + i * y_stride).
GemvArgs gemv_args(const mmhip_weight* w, uint64_t first, uint64_t n, const float* x, uint64_t x_stride, float* y,
                   uint64_t y_stride);
int qmm_device(mmhip_ctx* ctx, const mmhip_weight* w, uint64_t mat, const float* x, float* y,
               uint64_t batch, int out_layout, DevBuf* qscratch);
// Whether the batched matmul of w runs as one launch with the activation
// quantisation inside (Q8_0, K <= 2048, x below 2 GiB): then it needs no
// digit scratch.
bool qmm_fused(const mmhip_weight* w, uint64_t batch);

}  // namespace mmhip
