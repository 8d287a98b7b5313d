// Operator planner: OpScheduler.planLayer and LayerPlan (src/scheduler.zig:265-552)
// with the rules of this backend. Host logic only.
//
// Same as the reference:
//   attn_norm, ffn_norm      -> CPU
//   attention                -> CPU (on the reference's blacklist; NPU otherwise)
//   heavy throttle           -> every FFN op on the CPU
//   estimates                -> perf-db cpu_us for (op, shape, precision), else
//                               fallbackEstimate (scheduler.zig:523-537), which
//                               reads only m and n: 1-D ops (norm, silu) get 0
// Added for the HIP backend (the GPU rules the reference leaves empty):
//   with a GPU, gate/up, silu*up and down run on the GPU (the NPU keeps gate/up
//   only when there is no GPU), and a perf-db gpu_us is used for GPU ops;
//   the FFN precision comes from the weights (Q8_0 or IQ2_XXS).
#include <algorithm>
#include <cstdint>
#include <cstring>

#include "../../include/mmhip.h"
#include "backend.hpp"

namespace {

struct Planner {
    bool has_gpu, has_npu;
    int level;
    const mmhip_perf_entry* db;
    size_t db_len;

    bool heavy() const { return level == 3; }

    const mmhip_perf_entry* query(uint32_t op, const mmhip_shape& s, uint32_t prec) const {
        for (size_t i = 0; i < db_len; ++i) {
            const mmhip_perf_entry& e = db[i];
            if (e.op == op && e.precision == prec && e.shape.m == s.m && e.shape.n == s.n && e.shape.k == s.k &&
                e.shape.dim == s.dim)
                return &e;
        }
        return nullptr;
    }

    // fallbackEstimate (scheduler.zig:523-537), in 64-bit arithmetic.
    static uint64_t fallback(uint32_t op, const mmhip_shape& s) {
        const uint64_t dim = std::max(s.m, s.n), m = s.m, n = s.n, k = s.k;
        switch (op) {
            case MMHIP_OP_RMSNORM: return dim / 40;
            case MMHIP_OP_MATVEC_Q8_0: return m * k / 40000;
            case MMHIP_OP_MATMUL_Q8_0: return m * n * k / 8000000;
            case MMHIP_OP_SILU_MUL: return dim / 80;
            case MMHIP_OP_ATTENTION: return m * n * k / 2000000;
            case MMHIP_OP_FFN_GATE_UP: return m * k / 40000;
            case MMHIP_OP_FFN_DOWN: return m * k / 35000;
            default: return 100;
        }
    }

    // queryEstUs (505-513), plus the GPU time when the op runs on the GPU.
    uint64_t est(uint32_t op, const mmhip_shape& s, uint32_t prec, uint32_t backend) const {
        if (const mmhip_perf_entry* e = query(op, s, prec)) {
            if (backend == MMHIP_BACKEND_GPU && e->gpu_us > 0) return e->gpu_us;
            return e->cpu_us;
        }
        return fallback(op, s);
    }
};

mmhip_shape shape(uint32_t m, uint32_t n, uint32_t k, uint32_t dim) { return mmhip_shape{m, n, k, dim}; }

}  // namespace

extern "C" {

int mmhip_plan_layer(uint32_t layer, const mmhip_plan_hparams* hp, int has_gpu, int has_npu, int throttle_level,
                     const mmhip_perf_entry* db, size_t db_len, mmhip_op_schedule* out, size_t cap, size_t* n_out) {
    if (!hp || !n_out || (cap && !out) || (db_len && !db)) {
        mmhip::set_error(MMHIP_ERR_INVALID, "plan_layer: null argument");
        return MMHIP_ERR_INVALID;
    }
    const uint32_t wprec = hp->weight_precision;
    if (wprec != MMHIP_PREC_Q8_0 && wprec != MMHIP_PREC_IQ2_XXS) {
        mmhip::set_error(MMHIP_ERR_UNSUPPORTED, "plan_layer: FFN weights must be Q8_0 or IQ2_XXS");
        return MMHIP_ERR_UNSUPPORTED;
    }
    const Planner P{has_gpu != 0, has_npu != 0, throttle_level, db, db_len};
    mmhip_op_schedule ops[8];
    size_t n = 0;
    auto add = [&](uint32_t op, uint32_t backend, mmhip_shape s, uint32_t prec, uint32_t est_op, uint32_t est_prec,
                   bool sync) {
        mmhip_op_schedule& o = ops[n++];
        o.op = op;
        o.backend = backend;
        o.precision = prec;
        o.sync_after = sync ? 1u : 0u;
        o.shape = s;
        o.estimated_us = P.est(est_op, s, est_prec, backend);
    };
    const uint32_t H = hp->hidden_size, I = hp->intermediate_size;
    const uint32_t seq = hp->seq_len_hint ? hp->seq_len_hint : 128;
    const bool dense = layer < hp->leading_dense_layers || hp->n_routed_experts <= 1;

    // 1. attn_norm, 2. attention (blacklisted to the CPU), 3. ffn_norm.
    add(MMHIP_OP_RMSNORM, MMHIP_BACKEND_CPU, shape(0, 0, 0, H), MMHIP_PREC_F32, MMHIP_OP_RMSNORM, MMHIP_PREC_F32,
        false);
    add(MMHIP_OP_ATTENTION, MMHIP_BACKEND_CPU, shape(hp->num_heads, hp->head_dim, seq, 0), MMHIP_PREC_F32,
        MMHIP_OP_ATTENTION, MMHIP_PREC_F32, false);
    add(MMHIP_OP_RMSNORM, MMHIP_BACKEND_CPU, shape(0, 0, 0, H), MMHIP_PREC_F32, MMHIP_OP_RMSNORM, MMHIP_PREC_F32,
        false);

    // 4. FFN (dense, or the MoE layer's shared expert; the routed experts are
    // placed by Scheduler.route).
    uint32_t gate = MMHIP_BACKEND_CPU;
    if (!P.heavy()) {
        if (P.has_gpu) gate = MMHIP_BACKEND_GPU;
        else if (P.has_npu) gate = MMHIP_BACKEND_NPU;
    }
    const uint32_t silu = dense ? (gate == MMHIP_BACKEND_NPU ? MMHIP_BACKEND_CPU : gate)
                                : (gate == MMHIP_BACKEND_GPU ? MMHIP_BACKEND_GPU : MMHIP_BACKEND_CPU);
    const uint32_t down = (P.has_gpu && !P.heavy()) ? MMHIP_BACKEND_GPU : MMHIP_BACKEND_CPU;
    add(MMHIP_OP_FFN_GATE_UP, gate, shape(I, 0, H, 0), wprec, MMHIP_OP_MATVEC_Q8_0, wprec,
        gate != MMHIP_BACKEND_CPU && gate != silu);
    add(MMHIP_OP_SILU_MUL, silu, shape(0, 0, 0, I), MMHIP_PREC_F32, MMHIP_OP_SILU_MUL, MMHIP_PREC_F32, false);
    add(MMHIP_OP_FFN_DOWN, down, shape(H, 0, I, 0), wprec, MMHIP_OP_MATVEC_Q8_0, wprec, true);

    *n_out = n;
    if (cap < n) {
        mmhip::set_error(MMHIP_ERR_INVALID, "plan_layer: output holds fewer than the plan's ops");
        return MMHIP_ERR_INVALID;
    }
    std::memcpy(out, ops, n * sizeof(mmhip_op_schedule));
    return MMHIP_OK;
}

// LayerPlan.estimatedCriticalPathUs (313-333): ops between sync points form a
// group; ops of one backend add up, ops on another backend overlap (max).
uint64_t mmhip_plan_critical_path_us(const mmhip_op_schedule* ops, size_t n) {
    uint64_t total = 0, group = 0;
    bool have = false;
    uint32_t current = 0;
    for (size_t i = 0; i < n; ++i) {
        const mmhip_op_schedule& o = ops[i];
        if (!have || o.sync_after) {
            total += group;
            group = o.estimated_us;
            current = o.backend;
            have = true;
        } else if (o.backend == current) {
            group += o.estimated_us;
        } else {
            group = std::max(group, o.estimated_us);
        }
    }
    return total + group;
}

// LayerPlan.deviceMask (336-346): bit 0 CPU, 1 GPU, 2 NPU.
uint32_t mmhip_plan_device_mask(const mmhip_op_schedule* ops, size_t n) {
    uint32_t mask = 0;
    for (size_t i = 0; i < n; ++i) mask |= 1u << ops[i].backend;
    return mask;
}

}  // extern "C"
