// MoE FFN layer on the device: the role of moeFFN (src/inference.zig:886-1010)
// with expertFFN (1152-1188), sharedExpertFFN (1094-1146), Scheduler.route
// (src/scheduler.zig:169-262) and forwardBatch's per-token loop (346-351).
//
// One call enqueues, on the context stream:
//   T == 1 with IQ2_XXS experts (shared expert merged or absent): the whole
//   layer as one cooperative launch (decode_moe.hip)          "moe_decode"
//   otherwise:
//   router scores   f32/f16 GEMV, [T][E]                     "moe_router"
//   T > 1: route    heap top-k, softmax, throttle, counts,
//                   slot layout and problem lists            "moe_route"
//   T == 1 (decode):
//     gate/up       quantised GEMV over the routed (+ shared)
//                   experts' gate and up matrices; every
//                   workgroup routes the token itself and one
//                   writes the routing outputs               "moe_gateup"
//     down          quantised GEMV, input silu(gate) * up
//                   formed while quantising; with IQ2_XXS
//                   experts (shared merged) it also does the
//                   combine in the same launch               "moe_down"
//   T > 1 (prefill, experts grouped):
//     quantise hidden (with IQ2_XXS experts: inside the
//     routing launch)                                         "moe_quantize"
//     gate/up       grouped QMM over expert-sorted slots      "moe_gateup"
//     silu*up       quantised per slot                        "moe_quantize"
//     down          grouped QMM                               "moe_down"
//   combine         weighted sum in route order + shared
//                   + deferral bias                           "moe_combine"
// No routing result returns to the host in between.
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>

#include "../../include/mmhip.h"
#include "backend.hpp"

using namespace mmhip;

struct mmhip_moe_layer {
    uint32_t hidden = 0, inter = 0, shared_inter = 0, n_experts = 0;
    uint32_t expert_type = 0, shared_type = 0, router_type = 0;
    float rsf = 1.0f;
    bool has_shared = false, shared_merged = false;
    mmhip_weight* router = nullptr;  // [E][H], count 1
    mmhip_weight* gu = nullptr;      // gate 0..E-1, up E..2E-1 (+ shared gate 2E, up 2E+1 when merged)
    mmhip_weight* dn = nullptr;      // down 0..E-1 (+ shared down E when merged)
    mmhip_weight* sh_gu = nullptr;   // shared gate, up (not merged)
    mmhip_weight* sh_dn = nullptr;
    unsigned long long* counts = nullptr;  // device [E]
    uint32_t max_work = 0;
    std::mutex mu;
    // Device scratch, one allocation, sized for MMHIP_MOE_MAX_TOKENS tokens.
    void* scratch = nullptr;
    float* scores = nullptr;
    int32_t* assign_slot = nullptr;
    float* assign_w = nullptr;
    int32_t* shared_slot = nullptr;
    uint32_t* deferred = nullptr;
    uint32_t* slot_tok = nullptr;
    uint4* gemv_gu = nullptr;
    uint4* gemv_dn = nullptr;
    uint32_t* n_gemv = nullptr;
    QmmWork* work_gu = nullptr;
    QmmWork* work_dn = nullptr;
    uint32_t* n_work = nullptr;
    uint32_t* route_ids = nullptr;
    float* route_w = nullptr;
    float* y_gu = nullptr;   // [5 T][2 inter]
    float* y_sh = nullptr;   // [T][2 shared_inter] (shared not merged)
    float* eo = nullptr;     // [5 T][hidden]
    void* xq_h = nullptr;    // quantised hidden [T][gu cols_pad]
    void* xq_d = nullptr;    // quantised down input [5 T][dn cols_pad]
    void* xq_sd = nullptr;   // quantised shared down input [T][sh_dn cols_pad]
    float* bias = nullptr;   // [hidden]
    // One-launch decode (IQ2_XXS experts): h planes and scales handed from
    // the gate/up workgroups to the down workgroups, and the grid counters.
    uint8_t* dm_hq = nullptr;   // [5][inter / 32][64]
    float* dm_hs = nullptr;     // [5][inter / 32]
    uint64_t* dm_scores = nullptr;  // [n_experts] epoch-tagged router scores
    uint32_t* dm_flags = nullptr;   // [5][inter / 32] epoch-tagged h blocks
    uint32_t dm_epoch = 0;          // number of the last one-launch call (never 0 once called)
    bool decode_fused = false;  // the layer's decode calls use the one-launch kernel
    uint32_t dm_wait_ticks = 0;  // 10 ns ticks before a grid-wide wait gives up
    float* d_in = nullptr;   // host-ABI staging [T][hidden]
    float* d_out = nullptr;
};

namespace {

constexpr uint32_t kMaxTok = MMHIP_MOE_MAX_TOKENS;

uint64_t align256(uint64_t v) { return (v + 255) / 256 * 256; }

// ThrottleState.throttle (thermal.zig:44-72): active expert limit per level.
uint32_t level_limit(int level) {
    static const uint32_t limit[4] = {4, 3, 2, 1};
    return limit[level];
}

// getRoutedScalingFactor (scheduler.zig:254-262), in f32 as the CPU path.
float routed_scale(int level, float rsf) {
    switch (level) {
        case 1: return rsf * 0.83f;
        case 2: return rsf * 0.67f;
        case 3: return rsf * 0.5f;
        default: return rsf;
    }
}

void layer_free(mmhip_moe_layer* L) {
    weight_destroy(L->router);
    weight_destroy(L->gu);
    weight_destroy(L->dn);
    weight_destroy(L->sh_gu);
    weight_destroy(L->sh_dn);
    if (L->counts) (void)hipFree(L->counts);
    if (L->scratch) (void)hipFree(L->scratch);
    delete L;
}

bool quantised(uint32_t t) { return t == kQ8_0 || t == kIq2Xxs; }

// Carves the scratch allocation; returns its size (base may be null to size).
size_t carve(mmhip_moe_layer* L, char* base) {
    const uint64_t T = kMaxTok, S = 5 * kMaxTok, H = L->hidden, I = L->inter;
    uint64_t off = 0;
    auto take = [&](uint64_t bytes) -> char* {
        char* p = base ? base + off : nullptr;
        off += align256(bytes);
        return p;
    };
    L->scores = (float*)take(T * L->n_experts * 4);
    L->assign_slot = (int32_t*)take(T * 4 * 4);
    L->assign_w = (float*)take(T * 4 * 4);
    L->shared_slot = (int32_t*)take(T * 4);
    L->deferred = (uint32_t*)take(T * 4);
    L->slot_tok = (uint32_t*)take(S * 4);
    L->gemv_gu = (uint4*)take(10 * 16);
    L->gemv_dn = (uint4*)take(5 * 16);
    L->n_gemv = (uint32_t*)take(2 * 4);
    L->work_gu = (QmmWork*)take((uint64_t)L->max_work * sizeof(QmmWork));
    L->work_dn = (QmmWork*)take((uint64_t)L->max_work * sizeof(QmmWork));
    L->n_work = (uint32_t*)take(2 * 4);
    L->route_ids = (uint32_t*)take(T * 4 * 4);
    L->route_w = (float*)take(T * 4 * 4);
    L->y_gu = (float*)take(S * 2 * I * 4);
    if (L->has_shared && !L->shared_merged) L->y_sh = (float*)take(T * 2 * L->shared_inter * 4);
    L->eo = (float*)take(S * H * 4);
    L->xq_h = take(quant_act_bytes(T, L->gu->geom.cols_pad));
    L->xq_d = take(quant_act_bytes(S, L->dn->geom.cols_pad));
    if (L->has_shared && !L->shared_merged) L->xq_sd = take(quant_act_bytes(T, L->sh_dn->geom.cols_pad));
    L->bias = (float*)take(H * 4);
    L->dm_hq = (uint8_t*)take(5 * (uint64_t)(I / 32) * 64);
    L->dm_hs = (float*)take(5 * (uint64_t)(I / 32) * 4);
    L->dm_scores = (uint64_t*)take((uint64_t)L->n_experts * 8);
    L->dm_flags = (uint32_t*)take(5 * (uint64_t)(I / 32) * 4);
    L->d_in = (float*)take(T * H * 4);
    L->d_out = (float*)take(T * H * 4);
    return off;
}

int gemv_launch(mmhip_ctx* ctx, const mmhip_weight* w, const char* family, const uint4* probs, const uint32_t* n_active,
                uint32_t n_probs, const float* x, uint64_t x_stride, uint64_t x2_off, bool silu, float* y,
                uint64_t y_stride, const RouteArgs* route = nullptr) {
    const TileGeom& g = w->geom;
    GemvArgs a{};
    a.recs = w->recs;
    a.dvals = w->dvals;
    a.rec_stride = g.rec_stride;
    a.d_stride = g.d_stride;
    a.d_row = (uint32_t)g.d_row;
    a.x = x;
    a.x_stride = x_stride;
    a.x2_off = x2_off;
    a.silu_mul = silu ? 1u : 0u;
    a.y = y;
    a.y_stride = y_stride;
    a.first_mat = 0;
    a.probs = probs;
    a.n_active = n_active;
    a.n_probs = n_probs;
    a.tiles = (uint32_t)g.tiles;
    a.units = (uint32_t)g.units;
    a.rows = (uint32_t)g.rows;
    a.cols = (uint32_t)g.cols;
    if (route) {
        a.route = *route;
        a.route_decode = 1;
    }
    hipError_t e;
    {
        TimedLaunch tl(ctx, family);
        e = launch_gemv_q(a, g.fmt, ctx->num_cu, ctx->stream);
    }
    return e == hipSuccess ? MMHIP_OK : hip_fail(e, family);
}

#define MOE_TRY(expr)               \
    do {                            \
        const int rc_ = (expr);     \
        if (rc_ != MMHIP_OK) return rc_; \
    } while (0)

int check_hip(hipError_t e, const char* what) { return e == hipSuccess ? MMHIP_OK : hip_fail(e, what); }

// The device sequence of one call; T in [1, kMaxTok].
int ffn_enqueue(mmhip_ctx* ctx, mmhip_moe_layer* L, const float* hidden, float* out, uint32_t T, int level, uint32_t k,
                bool with_bias, uint32_t* route_ids, float* route_w) {
    const uint32_t H = L->hidden, I = L->inter, E = L->n_experts;
    hipStream_t s = ctx->stream;
    RouteArgs r{};
    r.scores = L->scores;
    r.n_tokens = T;
    r.n_experts = E;
    r.k = k;
    r.level = level;
    r.scale = routed_scale(level, L->rsf);
    r.shared = L->has_shared ? 1u : 0u;
    r.shared_merged = L->shared_merged ? 1u : 0u;
    r.counts = L->counts;
    r.route_ids = route_ids;
    r.route_w = route_w;
    r.assign_slot = L->assign_slot;
    r.assign_w = L->assign_w;
    r.shared_slot = L->shared_slot;
    r.deferred = L->deferred;
    r.slot_tok = L->slot_tok;
    r.gemv_gu = L->gemv_gu;
    r.gemv_dn = L->gemv_dn;
    r.n_gemv = L->n_gemv;
    r.work_gu = L->work_gu;
    r.work_dn = L->work_dn;
    r.n_work = L->n_work;
    r.inter = I;
    const bool fused = T == 1 && L->decode_fused;
    if (!fused) {
        TimedLaunch tl(ctx, "moe_router");
        MOE_TRY(check_hip(launch_gemv_float(L->router->plain, L->router_type, 0, hidden, H, L->scores, E, T, E, H, s),
                          "moe: router"));
    }
    const bool sep_shared = L->has_shared && !L->shared_merged;
    const uint32_t SI = L->shared_inter;
    // One activation scale per 256 columns when an IQ2_XXS grouped matmul
    // reads the hidden digits (routed experts or the shared expert); then the
    // routing launch also quantises them.
    const bool wide_h = L->gu->geom.fmt == kFmtIq2 || (sep_shared && L->sh_gu->geom.fmt == kFmtIq2);
    const QuantAct qh = quant_act_view(L->xq_h, T, L->gu->geom.cols_pad);
    if (T > 1) {
        if (wide_h) {
            r.qx = hidden;
            r.qx_stride = H;
            r.q_cols = H;
            r.q_units = (uint32_t)(L->gu->geom.cols_pad / 256);
            r.qa = qh;
        }
        TimedLaunch tl(ctx, "moe_route");
        MOE_TRY(check_hip(launch_route(r, s), "moe: route"));
    }
    if (fused) {
        // Decode in one launch: router, routing, gate/up, down and combine.
        const TileGeom& gg = L->gu->geom;
        const TileGeom& gd = L->dn->geom;
        DecodeMoeArgs d{};
        d.route = r;
        d.router_w = L->router->plain;
        d.router_type = L->router_type;
        d.x = hidden;
        d.hidden = H;
        d.inter = I;
        d.gu_recs = L->gu->recs;
        d.gu_dvals = L->gu->dvals;
        d.gu_rec_stride = gg.rec_stride;
        d.gu_d_stride = gg.d_stride;
        d.gu_d_row = (uint32_t)gg.d_row;
        d.dn_recs = L->dn->recs;
        d.dn_dvals = L->dn->dvals;
        d.dn_rec_stride = gd.rec_stride;
        d.dn_d_stride = gd.d_stride;
        d.dn_d_row = (uint32_t)gd.d_row;
        d.hq = L->dm_hq;
        d.hs = L->dm_hs;
        d.score_tags = L->dm_scores;
        d.h_flags = L->dm_flags;
        if (++L->dm_epoch == 0) L->dm_epoch = 1;
        d.epoch = L->dm_epoch;
        d.wait_ticks = L->dm_wait_ticks;
        d.status = ctx->status_dev;
        d.bias = with_bias ? L->bias : nullptr;
        d.out = out;
        TimedLaunch tl(ctx, "moe_decode");
        return check_hip(launch_decode_moe_iq2(d, ctx->num_cu, s), "moe: one-launch decode");
    }
    if (T == 1) {
        // Decode: the gate/up GEMV routes the token itself (no routing launch).
        MOE_TRY(gemv_launch(ctx, L->gu, "moe_gateup", nullptr, nullptr, L->shared_merged ? 10 : 8, hidden, 0, 0, false,
                            L->y_gu, I, &r));
        if (sep_shared)
            MOE_TRY(gemv_launch(ctx, L->sh_gu, "moe_gateup", nullptr, nullptr, 2, hidden, 0, 0, false, L->y_sh, SI));
        const TileGeom& gd = L->dn->geom;
        if (!sep_shared && gd.fmt == kFmtIq2 && gd.units <= 8) {
            // Down projection and combine in one launch.
            DownCombineArgs d{};
            d.recs = L->dn->recs;
            d.dvals = L->dn->dvals;
            d.rec_stride = gd.rec_stride;
            d.d_stride = gd.d_stride;
            d.d_row = (uint32_t)gd.d_row;
            d.probs = L->gemv_dn;
            d.n_active = L->n_gemv + 1;
            d.x = L->y_gu;
            d.x_stride = 2 * (uint64_t)I;
            d.x2_off = I;
            d.assign_slot = L->assign_slot;
            d.assign_w = L->assign_w;
            d.shared_slot = L->shared_slot;
            d.deferred = L->deferred;
            d.bias = with_bias ? L->bias : nullptr;
            d.out = out;
            d.tiles = (uint32_t)gd.tiles;
            d.units = (uint32_t)gd.units;
            d.rows = (uint32_t)gd.rows;
            d.cols = (uint32_t)gd.cols;
            TimedLaunch tl(ctx, "moe_down");
            return check_hip(launch_down_combine_iq2(d, s), "moe: down + combine");
        }
        MOE_TRY(gemv_launch(ctx, L->dn, "moe_down", L->gemv_dn, L->n_gemv + 1, 5, L->y_gu, 2 * (uint64_t)I, I, true,
                            L->eo, H));
        if (sep_shared)
            MOE_TRY(gemv_launch(ctx, L->sh_dn, "moe_down", nullptr, nullptr, 1, L->y_sh, 2 * (uint64_t)SI, SI, true,
                                L->eo + 4 * (uint64_t)H, H));
    } else {
        const TileGeom& gg = L->gu->geom;
        const TileGeom& gd = L->dn->geom;
        if (!wide_h) {
            TimedLaunch tl(ctx, "moe_quantize");
            MOE_TRY(check_hip(launch_quantize(hidden, H, T, H, (uint32_t)gg.cols_pad, qh, s, false), "moe: quantize"));
        }
        {
            TimedLaunch tl(ctx, "moe_gateup");
            MOE_TRY(check_hip(launch_group_experts(L->gu->recs, L->gu->dvals, gg, qh, L->slot_tok, L->work_gu, L->n_work,
                                                   route_max_work(T, E), L->y_gu, 2 * (uint64_t)I, ctx->num_cu, s),
                              "moe: gate/up"));
            if (sep_shared) {
                const TileGeom& gs = L->sh_gu->geom;
                if (gs.cols_pad != gg.cols_pad) {
                    set_error(MMHIP_ERR_UNSUPPORTED, "moe: shared gate/up padding differs from the routed experts'");
                    return MMHIP_ERR_UNSUPPORTED;
                }
                MOE_TRY(check_hip(launch_group_dense(L->sh_gu->recs, L->sh_gu->dvals, gs, 0, qh, T, L->y_sh,
                                                     2 * (uint64_t)SI, 0, ctx->num_cu, s),
                                  "moe: shared gate"));
                MOE_TRY(check_hip(launch_group_dense(L->sh_gu->recs, L->sh_gu->dvals, gs, 1, qh, T, L->y_sh + SI,
                                                     2 * (uint64_t)SI, 0, ctx->num_cu, s),
                                  "moe: shared up"));
            }
        }
        const QuantAct qd = quant_act_view(L->xq_d, 5 * (uint64_t)T, gd.cols_pad);
        {
            TimedLaunch tl(ctx, "moe_quantize");
            MOE_TRY(check_hip(launch_quantize_silu(L->y_gu, 2 * (uint64_t)I, I, nullptr, 5 * T, I, (uint32_t)gd.cols_pad,
                                                   qd, s, gd.fmt == kFmtIq2),
                              "moe: silu quantize"));
        }
        {
            TimedLaunch tl(ctx, "moe_down");
            MOE_TRY(check_hip(launch_group_experts(L->dn->recs, L->dn->dvals, gd, qd, nullptr, L->work_dn, L->n_work + 1,
                                                   route_max_work(T, E) / 2, L->eo, H, ctx->num_cu, s),
                              "moe: down"));
            if (sep_shared) {
                const TileGeom& gs = L->sh_dn->geom;
                const QuantAct qs = quant_act_view(L->xq_sd, T, gs.cols_pad);
                MOE_TRY(check_hip(launch_quantize_silu(L->y_sh, 2 * (uint64_t)SI, SI, nullptr, T, SI,
                                                       (uint32_t)gs.cols_pad, qs, s, gs.fmt == kFmtIq2),
                                  "moe: shared silu quantize"));
                MOE_TRY(check_hip(launch_group_dense(L->sh_dn->recs, L->sh_dn->dvals, gs, 0, qs, T,
                                                     L->eo + 4 * (uint64_t)T * H, H, 0, ctx->num_cu, s),
                                  "moe: shared down"));
            }
        }
    }
    {
        TimedLaunch tl(ctx, "moe_combine");
        MOE_TRY(check_hip(launch_combine(L->eo, L->assign_slot, L->assign_w, L->shared_slot, L->deferred,
                                         with_bias ? L->bias : nullptr, out, T, H, s),
                          "moe: combine"));
    }
    return MMHIP_OK;
}

// Validates the call and resolves (level, k).
int call_params(const mmhip_moe_layer* L, uint32_t T, const mmhip_route_params* rp, int* level, uint32_t* k) {
    if (T == 0 || T > kMaxTok) {
        set_error(MMHIP_ERR_INVALID, "moe: n_tokens must be in [1, " + std::to_string(kMaxTok) + "]");
        return MMHIP_ERR_INVALID;
    }
    const int lv = rp ? rp->throttle_level : 0;
    if (lv < 0 || lv > 3) {
        // ThrottleLevel has four values (thermal.zig:17-22); anything else is a
        // caller error, not a reason to run unthrottled.
        set_error(MMHIP_ERR_INVALID, "moe: throttle_level must be in [0, 3], got " + std::to_string(lv));
        return MMHIP_ERR_INVALID;
    }
    const uint32_t limit = (rp && rp->active_expert_limit) ? rp->active_expert_limit : level_limit(lv);
    uint32_t kk = limit < 4 ? limit : 4;
    if (kk > L->n_experts) kk = L->n_experts;
    if (kk == 0) {
        set_error(MMHIP_ERR_INVALID, "moe: route selected no expert");
        return MMHIP_ERR_INVALID;
    }
    *level = lv;
    *k = kk;
    return MMHIP_OK;
}

int upload_bias(mmhip_ctx* ctx, mmhip_moe_layer* L, const mmhip_route_params* rp, bool* with_bias) {
    *with_bias = rp && rp->deferral_bias_host;
    if (!*with_bias) return MMHIP_OK;
    return check_hip(hipMemcpyAsync(L->bias, rp->deferral_bias_host, (size_t)L->hidden * 4, hipMemcpyHostToDevice,
                                    ctx->stream),
                     "moe: deferral bias");
}

}  // namespace

extern "C" {

int mmhip_moe_layer_create(mmhip_ctx* ctx, const mmhip_moe_weights* wts, mmhip_moe_layer** out_layer) {
    if (!ctx || !wts || !out_layer) {
        set_error(MMHIP_ERR_INVALID, "moe_layer_create: null argument");
        return MMHIP_ERR_INVALID;
    }
    *out_layer = nullptr;
    const mmhip_moe_weights& w = *wts;
    if (!w.hidden_size || !w.moe_intermediate || !w.n_routed_experts || w.n_routed_experts > 256 || !w.router_host ||
        !w.expert_gate_host || !w.expert_up_host || !w.expert_down_host) {
        set_error(MMHIP_ERR_INVALID, "moe_layer_create: sizes must be > 0, n_routed_experts <= 256, weights non-null");
        return MMHIP_ERR_INVALID;
    }
    if (!quantised(w.expert_type) || (w.router_type != kF32 && w.router_type != kF16)) {
        set_error(MMHIP_ERR_UNSUPPORTED, "moe_layer_create: experts must be Q8_0 or IQ2_XXS, the router F32 or F16");
        return MMHIP_ERR_UNSUPPORTED;
    }
    const bool has_shared = w.shared_gate_host != nullptr;
    if (has_shared && (!w.shared_up_host || !w.shared_down_host || !w.shared_intermediate ||
                       !quantised(w.shared_type))) {
        set_error(MMHIP_ERR_INVALID, "moe_layer_create: shared expert needs gate, up, down, a width and Q8_0/IQ2_XXS");
        return MMHIP_ERR_INVALID;
    }
    (void)hipSetDevice(ctx->device);
    mmhip_moe_layer* L = new mmhip_moe_layer();
    L->hidden = w.hidden_size;
    L->inter = w.moe_intermediate;
    L->shared_inter = has_shared ? w.shared_intermediate : 0;
    L->n_experts = w.n_routed_experts;
    L->expert_type = w.expert_type;
    L->shared_type = w.shared_type;
    L->router_type = w.router_type;
    L->rsf = w.routed_scaling_factor;
    L->has_shared = has_shared;
    L->shared_merged = has_shared && w.shared_type == w.expert_type && w.shared_intermediate == w.moe_intermediate;
    const uint64_t E = L->n_experts, H = L->hidden, I = L->inter;
    std::lock_guard<std::mutex> lock(ctx->mu);  // the upload uses the context's staging buffer
    int rc = weight_create(ctx, w.router_host, false, w.router_type, E, H, 1, &L->router);
    if (rc == MMHIP_OK) {
        WeightSegment segs[4] = {{w.expert_gate_host, E}, {w.expert_up_host, E}, {w.shared_gate_host, 1},
                                 {w.shared_up_host, 1}};
        rc = weight_create_segments(ctx, segs, L->shared_merged ? 4 : 2, false, w.expert_type, I, H, &L->gu);
    }
    if (rc == MMHIP_OK) {
        WeightSegment segs[2] = {{w.expert_down_host, E}, {w.shared_down_host, 1}};
        rc = weight_create_segments(ctx, segs, L->shared_merged ? 2 : 1, false, w.expert_type, H, I, &L->dn);
    }
    if (rc == MMHIP_OK && has_shared && !L->shared_merged) {
        const uint64_t SI = L->shared_inter;
        WeightSegment segs[2] = {{w.shared_gate_host, 1}, {w.shared_up_host, 1}};
        rc = weight_create_segments(ctx, segs, 2, false, w.shared_type, SI, H, &L->sh_gu);
        if (rc == MMHIP_OK) rc = weight_create(ctx, w.shared_down_host, false, w.shared_type, H, SI, 1, &L->sh_dn);
    }
    if (rc != MMHIP_OK) {
        layer_free(L);
        return rc;
    }
    L->max_work = route_max_work(kMaxTok, L->n_experts);
    const size_t bytes = carve(L, nullptr);
    hipError_t e = hipMalloc(&L->scratch, bytes);
    if (e == hipSuccess) e = hipMalloc(&L->counts, E * sizeof(unsigned long long));
    if (e == hipSuccess) e = hipMemsetAsync(L->counts, 0, E * sizeof(unsigned long long), ctx->stream);
    if (e == hipSuccess) e = hipMemsetAsync(L->scratch, 0, bytes, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) {
        layer_free(L);
        return hip_fail(e, "moe_layer_create: scratch");
    }
    carve(L, static_cast<char*>(L->scratch));
    // Decode calls run as one launch when the experts are IQ2_XXS, the
    // shared expert (if any) is merged, and the shapes fit the kernel;
    // MMHIP_DECODE_FUSED=0 selects the three-launch sequence instead.
    const char* fused_env = getenv("MMHIP_DECODE_FUSED");
    L->decode_fused = !(fused_env && fused_env[0] == '0') && L->gu->geom.fmt == kFmtIq2 &&
                      L->dn->geom.fmt == kFmtIq2 && (!has_shared || L->shared_merged) &&
                      decode_moe_iq2_fits(L->hidden, L->inter, L->n_experts, ctx->num_cu);
    // MMHIP_DECODE_WAIT_US=n: a grid-wide wait gives up n microseconds after
    // its first poll (0: after the first poll) and the call reports an error
    // (tests force the failure path with 0). At most 40 s.
    const char* wait_env = getenv("MMHIP_DECODE_WAIT_US");
    const unsigned long wait_us = wait_env ? strtoul(wait_env, nullptr, 10) : kDecodeWaitUs;
    L->dm_wait_ticks = (uint32_t)(wait_us < 40000000ul ? wait_us : 40000000ul) * 100u;  // 100 MHz ticks
    *out_layer = L;
    return MMHIP_OK;
}

void mmhip_moe_layer_destroy(mmhip_ctx* ctx, mmhip_moe_layer* layer) {
    if (!layer) return;
    if (ctx) {
        (void)hipSetDevice(ctx->device);
        (void)hipStreamSynchronize(ctx->stream);
    }
    layer_free(layer);
}

int mmhip_moe_ffn_dev(mmhip_ctx* ctx, mmhip_moe_layer* layer, const float* hidden_dev, float* out_dev,
                      uint32_t n_tokens, const mmhip_route_params* rp, uint32_t* route_ids_dev,
                      float* route_weights_dev) {
    if (!ctx || !layer || !hidden_dev || !out_dev) {
        set_error(MMHIP_ERR_INVALID, "moe_ffn_dev: null argument");
        return MMHIP_ERR_INVALID;
    }
    int level;
    uint32_t k;
    int rc = call_params(layer, n_tokens, rp, &level, &k);
    if (rc != MMHIP_OK) return rc;
    std::lock_guard<std::mutex> lock(layer->mu);  // then the context: no caller takes them in the other order
    std::lock_guard<std::mutex> ctx_lock(ctx->mu);
    (void)hipSetDevice(ctx->device);
    bool with_bias;
    rc = upload_bias(ctx, layer, rp, &with_bias);
    if (rc != MMHIP_OK) return rc;
    return ffn_enqueue(ctx, layer, hidden_dev, out_dev, n_tokens, level, k, with_bias, route_ids_dev,
                       route_weights_dev);
}

int mmhip_moe_ffn(mmhip_ctx* ctx, mmhip_moe_layer* layer, const float* hidden_host, float* out_host,
                  uint32_t n_tokens, const mmhip_route_params* rp, uint32_t* route_ids_host,
                  float* route_weights_host) {
    if (!ctx || !layer || !hidden_host || !out_host) {
        set_error(MMHIP_ERR_INVALID, "moe_ffn: null argument");
        return MMHIP_ERR_INVALID;
    }
    int level;
    uint32_t k;
    int rc = call_params(layer, n_tokens, rp, &level, &k);
    if (rc != MMHIP_OK) return rc;
    std::lock_guard<std::mutex> lock(layer->mu);  // then the context: no caller takes them in the other order
    std::lock_guard<std::mutex> ctx_lock(ctx->mu);
    (void)hipSetDevice(ctx->device);
    const size_t bytes = (size_t)n_tokens * layer->hidden * 4;
    hipStream_t s = ctx->stream;
    rc = check_hip(hipMemcpyAsync(layer->d_in, hidden_host, bytes, hipMemcpyHostToDevice, s), "moe_ffn: upload");
    bool with_bias = false;
    if (rc == MMHIP_OK) rc = upload_bias(ctx, layer, rp, &with_bias);
    if (rc == MMHIP_OK)
        rc = ffn_enqueue(ctx, layer, layer->d_in, layer->d_out, n_tokens, level, k, with_bias, layer->route_ids,
                         layer->route_w);
    if (rc == MMHIP_OK)
        rc = check_hip(hipMemcpyAsync(out_host, layer->d_out, bytes, hipMemcpyDeviceToHost, s), "moe_ffn: download");
    if (rc == MMHIP_OK && route_ids_host)
        rc = check_hip(hipMemcpyAsync(route_ids_host, layer->route_ids, (size_t)n_tokens * 16, hipMemcpyDeviceToHost, s),
                       "moe_ffn: route ids");
    if (rc == MMHIP_OK && route_weights_host)
        rc = check_hip(hipMemcpyAsync(route_weights_host, layer->route_w, (size_t)n_tokens * 16, hipMemcpyDeviceToHost,
                                      s),
                       "moe_ffn: route weights");
    const hipError_t e = hipStreamSynchronize(s);
    if (rc == MMHIP_OK && e != hipSuccess) rc = hip_fail(e, "moe_ffn: synchronize");
    if (rc == MMHIP_OK) rc = check_device_status(ctx, "moe_ffn");
    if (rc == MMHIP_OK && ctx->timer.on) ctx->timer.drain();
    return rc == MMHIP_OK ? (int)k : rc;
}

int mmhip_moe_expert_counts(mmhip_ctx* ctx, mmhip_moe_layer* layer, uint64_t* counts_host) {
    if (!ctx || !layer || !counts_host) {
        set_error(MMHIP_ERR_INVALID, "moe_expert_counts: null argument");
        return MMHIP_ERR_INVALID;
    }
    std::lock_guard<std::mutex> lock(layer->mu);  // then the context: no caller takes them in the other order
    std::lock_guard<std::mutex> ctx_lock(ctx->mu);
    (void)hipSetDevice(ctx->device);
    hipError_t e = hipMemcpyAsync(counts_host, layer->counts, (size_t)layer->n_experts * 8, hipMemcpyDeviceToHost,
                                  ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    return e == hipSuccess ? MMHIP_OK : hip_fail(e, "moe_expert_counts");
}

}  // extern "C"
