// HIP backend for the quantized-weight matrix path (MI355X / gfx950).
//
// Zig side of libmmhip (include/mmhip.h). It takes the place the OpenCL and
// Metal backends hold in the engine: same object shape as OpenCLBackend
// (isAvailable / init / deinit / op methods on host slices,
// src/opencl_backend.zig:55-537), same C-bridge conventions as
// metal_backend.zig (extern fn, status codes mapped to Zig errors,
// src/metal_backend.zig:7-46). Place this file next to inference.zig and link
// with linkSystemLibrary("mmhip") and linkSystemLibrary("amdhip64").
//
// Every compute method returns an error when the device is unusable; the
// caller keeps the reference's CPU fallback (src/inference.zig:1209-1213).

const std = @import("std");
const gguf = @import("gguf.zig");
const dequant = @import("dequant.zig");
const scheduler = @import("scheduler.zig");

// ---- C ABI (include/mmhip.h) ----

pub const Ctx = opaque {};
pub const Weight = opaque {};
pub const MoeLayerHandle = opaque {};
pub const GgufHandle = opaque {};

pub const MoeWeights = extern struct {
    hidden_size: u32,
    moe_intermediate: u32,
    shared_intermediate: u32,
    n_routed_experts: u32,
    expert_type: u32,
    shared_type: u32,
    router_type: u32,
    routed_scaling_factor: f32,
    router_host: ?*const anyopaque,
    expert_gate_host: ?*const anyopaque,
    expert_up_host: ?*const anyopaque,
    expert_down_host: ?*const anyopaque,
    shared_gate_host: ?*const anyopaque = null,
    shared_up_host: ?*const anyopaque = null,
    shared_down_host: ?*const anyopaque = null,
};

pub const RouteParams = extern struct {
    throttle_level: i32 = 0,
    active_expert_limit: u32 = 0,
    deferral_bias_host: ?[*]const f32 = null,
};

pub const GemvGroup = extern struct {
    w: ?*const Weight,
    first: u64,
    n_mats: u64,
    x_dev: ?[*]const f32,
    x_stride: u64,
    y_dev: ?[*]f32,
    y_stride: u64,
};

pub const Shape = extern struct { m: u32 = 0, n: u32 = 0, k: u32 = 0, dim: u32 = 0 };

pub const OpSchedule = extern struct {
    op: u32,
    backend: u32,
    precision: u32,
    sync_after: u32,
    shape: Shape,
    estimated_us: u64,
};

pub const PlanHyperParams = extern struct {
    hidden_size: u32,
    intermediate_size: u32,
    num_heads: u32,
    head_dim: u32,
    seq_len_hint: u32 = 0,
    leading_dense_layers: u32,
    n_routed_experts: u32,
    weight_precision: u32,
};

pub const PerfEntry = extern struct {
    op: u32,
    precision: u32,
    shape: Shape,
    cpu_us: u64,
    gpu_us: u64,
};

pub const GgufInfo = extern struct {
    version: u32 = 0,
    tensor_count: u64 = 0,
    metadata_count: u64 = 0,
    n_tensors: u64 = 0,
    n_keys: u64 = 0,
    alignment: u64 = 0,
    data_offset: u64 = 0,
    file_size: u64 = 0,
};

pub const GgufTensor = extern struct {
    name: ?[*:0]const u8 = null,
    n_dims: u32 = 0,
    dims: [4]u64 = .{ 1, 1, 1, 1 },
    type_: u32 = 0,
    offset: u64 = 0,
    n_elements: u64 = 0,
    n_bytes: u64 = 0,
    data: ?*const anyopaque = null,
};

pub const max_moe_tokens: u32 = 256;

extern fn mmhip_last_error() [*:0]const u8;
extern fn mmhip_is_available() c_int;
extern fn mmhip_device_count() c_int;
extern fn mmhip_version() [*:0]const u8;
extern fn mmhip_init(out_ctx: *?*Ctx, device: c_int) c_int;
extern fn mmhip_destroy(ctx: ?*Ctx) void;
extern fn mmhip_synchronize(ctx: *Ctx) c_int;
extern fn mmhip_stream(ctx: *Ctx) ?*anyopaque;
extern fn mmhip_num_cu(ctx: *Ctx) c_int;
extern fn mmhip_profile_enable(ctx: *Ctx, enable: c_int) c_int;
extern fn mmhip_profile_read(ctx: *Ctx, family: [*:0]const u8, total_ms: *f64, launches: *u64) c_int;
extern fn mmhip_malloc(ctx: *Ctx, out_dev: *?*anyopaque, bytes: usize) c_int;
extern fn mmhip_free(ctx: *Ctx, dev: ?*anyopaque) c_int;
extern fn mmhip_memcpy_h2d(ctx: *Ctx, dst_dev: ?*anyopaque, src_host: ?*const anyopaque, bytes: usize) c_int;
extern fn mmhip_memcpy_d2h(ctx: *Ctx, dst_host: ?*anyopaque, src_dev: ?*const anyopaque, bytes: usize) c_int;
extern fn mmhip_memset_dev(ctx: *Ctx, dst_dev: ?*anyopaque, value: c_int, bytes: usize) c_int;
extern fn mmhip_gguf_open(path: [*:0]const u8, out: *?*GgufHandle) c_int;
extern fn mmhip_gguf_close(g: ?*GgufHandle) void;
extern fn mmhip_gguf_get_info(g: *const GgufHandle, out: *GgufInfo) c_int;
extern fn mmhip_gguf_tensor_at(g: *const GgufHandle, index: u64, out: *GgufTensor) c_int;
extern fn mmhip_gguf_find_tensor(g: *const GgufHandle, name: [*:0]const u8, out: *GgufTensor) c_int;
extern fn mmhip_gguf_key_at(g: *const GgufHandle, index: u64) ?[*:0]const u8;
extern fn mmhip_gguf_meta_type(g: *const GgufHandle, key: [*:0]const u8) c_int;
extern fn mmhip_gguf_meta_int(g: *const GgufHandle, key: [*:0]const u8, out: *i64) c_int;
extern fn mmhip_gguf_meta_float(g: *const GgufHandle, key: [*:0]const u8, out: *f64) c_int;
extern fn mmhip_gguf_meta_string(g: *const GgufHandle, key: [*:0]const u8, str: *?[*]const u8, len: *u64) c_int;
extern fn mmhip_gguf_meta_array(g: *const GgufHandle, key: [*:0]const u8, elem_type: *u32, len: *u64, data: *?*const anyopaque, n_bytes: *u64) c_int;
extern fn mmhip_weight_upload_gguf(ctx: *Ctx, g: *const GgufHandle, name: [*:0]const u8, out_w: *?*Weight) c_int;
extern fn mmhip_weight_upload_gguf_rows(ctx: *Ctx, g: *const GgufHandle, names: [*]const [*:0]const u8, n: u32, out_w: *?*Weight) c_int;
extern fn mmhip_moe_layer_create_gguf(ctx: *Ctx, g: *const GgufHandle, layer: u32, out_layer: *?*MoeLayerHandle) c_int;
extern fn mmhip_weight_upload(ctx: *Ctx, raw_host: ?*const anyopaque, type_: u32, rows: u64, cols: u64, count: u64, out_w: *?*Weight) c_int;
extern fn mmhip_weight_from_device(ctx: *Ctx, raw_dev: ?*const anyopaque, type_: u32, rows: u64, cols: u64, count: u64, out_w: *?*Weight) c_int;
extern fn mmhip_weight_free(ctx: *Ctx, w: ?*Weight) void;
extern fn mmhip_weight_device_bytes(w: *const Weight) u64;
extern fn mmhip_mat_vec_mul(ctx: *Ctx, out_host: [*]f32, ptr_host: ?*const anyopaque, type_: u32, x_host: [*]const f32, out_dim: u64, in_dim: u64) c_int;
extern fn mmhip_batch_mat_mul(ctx: *Ctx, out_host: [*]f32, ptr_host: ?*const anyopaque, type_: u32, in_host: [*]const f32, out_dim: u64, batch: u64, in_dim: u64) c_int;
extern fn mmhip_dequantize(ctx: *Ctx, out_host: [*]f32, data_host: ?*const anyopaque, type_: u32, n_elements: u64) c_int;
extern fn mmhip_forget(ctx: *Ctx, ptr_host: ?*const anyopaque) c_int;
extern fn mmhip_sample_greedy(ctx: *Ctx, out_host: *u32, logits_host: [*]const f32, n: u64) c_int;
extern fn mmhip_argmax_dev(ctx: *Ctx, out_dev: ?*u32, logits_dev: ?[*]const f32, n: u64) c_int;
extern fn mmhip_quantize_q8_0(ctx: *Ctx, blocks_host: ?*anyopaque, x_host: [*]const f32, n_elements: u64) c_int;
extern fn mmhip_quantize_q8_0_rows_dev(ctx: *Ctx, blocks_dev: ?*anyopaque, x_dev: ?[*]const f32, x_stride: u64, n_rows: u64, row_len: u32) c_int;
extern fn mmhip_dequantize_q8_0_rows_dev(ctx: *Ctx, out_dev: ?[*]f32, out_stride: u64, blocks_dev: ?*const anyopaque, n_rows: u64, row_len: u32) c_int;
extern fn mmhip_dequantize_dev(ctx: *Ctx, out_dev: ?[*]f32, raw_dev: ?*const anyopaque, type_: u32, n_elements: u64) c_int;
extern fn mmhip_gemv_dev(ctx: *Ctx, w: *const Weight, mat: u64, x_dev: ?[*]const f32, y_dev: ?[*]f32) c_int;
extern fn mmhip_gemv_batched_dev(ctx: *Ctx, w: *const Weight, first: u64, n_mats: u64, x_dev: ?[*]const f32, x_stride: u64, y_dev: ?[*]f32, y_stride: u64) c_int;
extern fn mmhip_gemv_grouped_dev(ctx: *Ctx, groups: [*]const GemvGroup, n_groups: u32) c_int;
extern fn mmhip_qmm_dev(ctx: *Ctx, w: *const Weight, mat: u64, x_dev: ?[*]const f32, y_dev: ?[*]f32, batch: u64, out_layout: c_int) c_int;
extern fn mmhip_qmm_dev_noalloc(ctx: *Ctx, w: *const Weight, mat: u64, x_dev: ?[*]const f32, y_dev: ?[*]f32, batch: u64, out_layout: c_int) c_int;
extern fn mmhip_moe_layer_create(ctx: *Ctx, wts: *const MoeWeights, out_layer: *?*MoeLayerHandle) c_int;
extern fn mmhip_moe_layer_destroy(ctx: *Ctx, layer: ?*MoeLayerHandle) void;
extern fn mmhip_moe_ffn(ctx: *Ctx, layer: *MoeLayerHandle, hidden_host: [*]const f32, out_host: [*]f32, n_tokens: u32, rp: ?*const RouteParams, route_ids_host: ?[*]u32, route_weights_host: ?[*]f32) c_int;
extern fn mmhip_moe_ffn_dev(ctx: *Ctx, layer: *MoeLayerHandle, hidden_dev: ?[*]const f32, out_dev: ?[*]f32, n_tokens: u32, rp: ?*const RouteParams, route_ids_dev: ?[*]u32, route_weights_dev: ?[*]f32) c_int;
extern fn mmhip_moe_expert_counts(ctx: *Ctx, layer: *MoeLayerHandle, counts_host: [*]u64) c_int;
extern fn mmhip_plan_layer(layer: u32, hp: *const PlanHyperParams, has_gpu: c_int, has_npu: c_int, throttle_level: c_int, db: ?[*]const PerfEntry, db_len: usize, out: [*]OpSchedule, cap: usize, n_out: *usize) c_int;
extern fn mmhip_plan_critical_path_us(ops: [*]const OpSchedule, n: usize) u64;
extern fn mmhip_plan_device_mask(ops: [*]const OpSchedule, n: usize) u32;

// ---- errors ----

pub const HipError = error{
    HipUnavailable,
    HipInvalidArgument,
    HipUnsupportedType,
    HipLaunch,
    HipOutOfMemory,
    HipNotFound,
};

fn check(rc: c_int) HipError!void {
    if (rc >= 0) return;
    std.log.debug("libmmhip: {s}", .{mmhip_last_error()});
    return switch (rc) {
        -1 => error.HipUnavailable,
        -2 => error.HipInvalidArgument,
        -3 => error.HipUnsupportedType,
        -5 => error.HipOutOfMemory,
        -6 => error.HipNotFound,
        else => error.HipLaunch,
    };
}

/// A gfx950 device is present and the library loaded (OpenCLBackend.isAvailable).
pub fn isAvailable() bool {
    return mmhip_is_available() == 1;
}

pub fn lastError() [*:0]const u8 {
    return mmhip_last_error();
}

// ---- backend object ----

pub const HipBackend = struct {
    ctx: *Ctx,
    allocator: std.mem.Allocator,

    const Self = @This();

    /// OpenCLBackend.init: one context on device 0.
    pub fn init(allocator: std.mem.Allocator) !Self {
        var ctx: ?*Ctx = null;
        try check(mmhip_init(&ctx, 0));
        return .{ .ctx = ctx.?, .allocator = allocator };
    }

    /// OpenCLBackend.deinit: frees the resident weights and the context.
    pub fn deinit(self: *Self) void {
        mmhip_destroy(self.ctx);
    }

    /// matVecMulUnified (inference.zig:1200-1228) on the device: out = W . x
    /// for Q8_0 / IQ2_XXS / F32 / F16 weights given as mmap'd GGUF bytes.
    /// The weight is uploaded on first use and stays resident, keyed by its
    /// host address (getOrUploadMatBuffer's role).
    pub fn matVecMulUnified(self: *Self, out: []f32, ptr: [*]const u8, type_: gguf.GgmlType, x: []const f32, out_dim: usize, in_dim: usize) !void {
        std.debug.assert(out.len >= out_dim and x.len >= in_dim);
        try check(mmhip_mat_vec_mul(self.ctx, out.ptr, ptr, @intFromEnum(type_), x.ptr, out_dim, in_dim));
    }

    /// batchMatMulUnified (1231-1264): out [batch][out_dim].
    pub fn batchMatMulUnified(self: *Self, out: []f32, ptr: [*]const u8, type_: gguf.GgmlType, in: []const f32, out_dim: usize, batch: usize, in_dim: usize) !void {
        std.debug.assert(out.len >= out_dim * batch and in.len >= in_dim * batch);
        try check(mmhip_batch_mat_mul(self.ctx, out.ptr, ptr, @intFromEnum(type_), in.ptr, out_dim, batch, in_dim));
    }

    /// OpenCLBackend.matMulQ8_0 (opencl_backend.zig:412-453): a Q8_0 GEMV
    /// despite the name.
    pub fn matMulQ8_0(self: *Self, out: []f32, mat: []const u8, vec: []const f32, out_dim: u32, in_dim: u32) !void {
        try self.matVecMulUnified(out, mat.ptr, .q8_0, vec, out_dim, in_dim);
    }

    /// dequant.dequantize (dequant.zig:632-659) on the device, bit-exact.
    pub fn dequantize(self: *Self, out: []f32, data: [*]const u8, type_: gguf.GgmlType) !void {
        try check(mmhip_dequantize(self.ctx, out.ptr, data, @intFromEnum(type_), out.len));
    }

    /// Engine.sampleGreedy (inference.zig:376-386) on the device: the first
    /// index of the largest logit.
    pub fn sampleGreedy(self: *Self, logits: []const f32) !u32 {
        var id: u32 = 0;
        try check(mmhip_sample_greedy(self.ctx, &id, logits.ptr, logits.len));
        return id;
    }

    /// Several weights' GEMVs (e.g. the routed experts' gate/up and down
    /// products) in one launch; all weights of one quantised type. No
    /// reference counterpart: it replaces one matVecMulUnified per matrix
    /// (inference.zig:1171-1185) with one launch.
    pub fn gemvGroupedDev(self: *Self, groups: []const GemvGroup) !void {
        try check(mmhip_gemv_grouped_dev(self.ctx, groups.ptr, @intCast(groups.len)));
    }

    /// The batched QMM on device buffers with the library's fixed scratch:
    /// allocates nothing, for code under graph capture or in loops that must
    /// not allocate. No reference counterpart. batch x cols (rounded up to
    /// 256) x 2.125 bytes must fit the 4,456,448-byte scratch; calls that
    /// overlap on one device race.
    pub fn qmmDevNoAlloc(self: *Self, w: *const Weight, mat: u64, x_dev: [*]const f32, y_dev: [*]f32, batch: u64, out_layout: c_int) !void {
        try check(mmhip_qmm_dev_noalloc(self.ctx, w, mat, x_dev, y_dev, batch, out_layout));
    }

    /// sampleGreedy on device logits (e.g. computeLogits' GEMV output kept
    /// on the device); the id lands in device memory.
    pub fn argmaxDev(self: *Self, out_dev: *u32, logits_dev: [*]const f32, n: u64) !void {
        try check(mmhip_argmax_dev(self.ctx, out_dev, logits_dev, n));
    }

    /// dequant.quantizeQ8_0 (dequant.zig:98-130) on the device: `blocks`
    /// receives (data.len + 31) / 32 blocks (caller-owned, unlike the
    /// reference's allocating version).
    pub fn quantizeQ8_0(self: *Self, blocks: []dequant.BlockQ8_0, data: []const f32) !void {
        std.debug.assert(blocks.len == (data.len + 31) / 32);
        try check(mmhip_quantize_q8_0(self.ctx, blocks.ptr, data.ptr, data.len));
    }

    /// KVCache.put's Q8_0 branch (kv_cache.zig:289-349) for n_rows device
    /// rows at once (e.g. a prefill's kv_comp rows of kv_lora_rank values).
    pub fn quantizeRowsQ8_0Dev(self: *Self, blocks_dev: *anyopaque, x_dev: [*]const f32, x_stride: u64, n_rows: u64, row_len: u32) !void {
        try check(mmhip_quantize_q8_0_rows_dev(self.ctx, blocks_dev, x_dev, x_stride, n_rows, row_len));
    }

    /// getKVCompressed / getKPe's Q8_0 branch (kv_cache.zig:225-273) for
    /// n_rows device rows at once.
    pub fn dequantizeRowsQ8_0Dev(self: *Self, out_dev: [*]f32, out_stride: u64, blocks_dev: *const anyopaque, n_rows: u64, row_len: u32) !void {
        try check(mmhip_dequantize_q8_0_rows_dev(self.ctx, out_dev, out_stride, blocks_dev, n_rows, row_len));
    }

    /// Drops the resident copy of a weight (e.g. before unmapping the file).
    pub fn forget(self: *Self, ptr: [*]const u8) void {
        _ = mmhip_forget(self.ctx, ptr);
    }

    pub fn synchronize(self: *Self) !void {
        try check(mmhip_synchronize(self.ctx));
    }
};

// ---- MoE FFN layer (moeFFN + Scheduler.route on the device) ----

pub const MoeLayer = struct {
    backend: *HipBackend,
    handle: *MoeLayerHandle,
    hidden: u32,
    /// Set while a PlanDispatch owns the layer (PlanDispatch.bind): the
    /// plan's FFN ops then run the whole moeFFN, and a direct ffn call
    /// returns error.HipInvalidArgument, so no token's experts run twice.
    plan_bound: bool = false,

    /// Uploads one layer's router, routed experts and shared expert.
    pub fn create(backend: *HipBackend, w: MoeWeights) !MoeLayer {
        var h: ?*MoeLayerHandle = null;
        try check(mmhip_moe_layer_create(backend.ctx, &w, &h));
        return .{ .backend = backend, .handle = h.?, .hidden = w.hidden_size };
    }

    /// The same from blk.<layer>'s FFN tensors of a GGUF file opened by
    /// GgufFile.open (Model.bindLayer, model.zig:289-395); the file may be
    /// closed afterwards.
    pub fn fromGguf(backend: *HipBackend, file: *const GgufFile, layer: u32, hidden: u32) !MoeLayer {
        var h: ?*MoeLayerHandle = null;
        try check(mmhip_moe_layer_create_gguf(backend.ctx, file.handle, layer, &h));
        return .{ .backend = backend, .handle = h.?, .hidden = hidden };
    }

    pub fn destroy(self: *MoeLayer) void {
        mmhip_moe_layer_destroy(self.backend.ctx, self.handle);
    }

    /// moeFFN for n tokens (hidden / out: [n][hidden]); route ids and weights
    /// ([n][4]) as Scheduler.route returns them. Returns k.
    pub fn ffn(self: *MoeLayer, hidden: []const f32, out: []f32, n_tokens: u32, rp: RouteParams, route_ids: ?[]u32, route_weights: ?[]f32) !u32 {
        if (self.plan_bound) return error.HipInvalidArgument;
        return self.ffnUnbound(hidden, out, n_tokens, rp, route_ids, route_weights);
    }

    fn ffnUnbound(self: *MoeLayer, hidden: []const f32, out: []f32, n_tokens: u32, rp: RouteParams, route_ids: ?[]u32, route_weights: ?[]f32) !u32 {
        std.debug.assert(n_tokens >= 1 and n_tokens <= max_moe_tokens);
        std.debug.assert(hidden.len >= n_tokens * self.hidden and out.len >= n_tokens * self.hidden);
        const rc = mmhip_moe_ffn(self.backend.ctx, self.handle, hidden.ptr, out.ptr, n_tokens, &rp, if (route_ids) |r| r.ptr else null, if (route_weights) |r| r.ptr else null);
        try check(rc);
        return @intCast(rc);
    }

    /// ExpertStats.counts of this layer.
    pub fn expertCounts(self: *MoeLayer, counts: []u64) !void {
        try check(mmhip_moe_expert_counts(self.backend.ctx, self.handle, counts.ptr));
    }
};

// ---- plan dispatch (HeteroExecutor.dispatchGpu, hetero_executor.zig:154-159) ----

/// The GPU side of HeteroExecutor.executeLayer (hetero_executor.zig:88-127)
/// for the ops planLayer sends to .gpu on a MoE layer (scheduler.zig:473-501
/// plus this backend's GPU rule): ffn_gate_up, siluMul and ffn_down of the
/// layer's FFN. The device runs the whole moeFFN (router, Scheduler.route,
/// expert gate/up, SiLU x up, down, weighted sum and shared expert) in one
/// call, so ffn_gate_up issues it for the token in `hidden`, siluMul is
/// already done inside it, and ffn_down hands the result back as moeFFN does
/// (hidden <- ffn_out, inference.zig:1009; the caller adds the residual).
/// Ops this backend does not run (attention, RMSNorm, RoPE, or a dense
/// layer's FFN without a MoeLayer) return error.HipUnsupportedType, and the
/// executor keeps them on its CPU path.
/// The reference's plan for a MoE layer names only the shared expert's
/// gate/up, siluMul and down (scheduler.zig:466-501) and leaves the routed
/// experts to moeFFN; here the plan's FFN ops run the whole layer. A layer
/// therefore runs through exactly one path: bind() takes it for the plan
/// (moeFFN's direct MoeLayer.ffn then fails with error.HipInvalidArgument,
/// and so does a second bind), release() gives it back.
pub const PlanDispatch = struct {
    moe: ?*MoeLayer,
    /// [hidden_size] buffer owned by the caller: the FFN output between
    /// ffn_gate_up and ffn_down.
    ffn_out: []f32,
    route: RouteParams = .{},
    pending: bool = false,

    pub fn bind(moe: ?*MoeLayer, ffn_out: []f32, route: RouteParams) !PlanDispatch {
        if (moe) |L| {
            if (L.plan_bound) return error.HipInvalidArgument;
            L.plan_bound = true;
        }
        return .{ .moe = moe, .ffn_out = ffn_out, .route = route };
    }

    pub fn release(self: *PlanDispatch) void {
        if (self.moe) |L| L.plan_bound = false;
        self.moe = null;
        self.pending = false;
    }

    pub fn dispatchGpu(self: *PlanDispatch, op: scheduler.OpSchedule, hidden: []f32) !void {
        switch (op.op) {
            .ffn_gate_up => {
                const L = self.moe orelse return error.HipUnsupportedType;
                std.debug.assert(hidden.len == L.hidden and self.ffn_out.len == L.hidden);
                _ = try L.ffnUnbound(hidden, self.ffn_out, 1, self.route, null, null);
                self.pending = true;
            },
            // SiLU(gate) * up is formed on the device inside the FFN call.
            .siluMul => if (!self.pending) return error.HipInvalidArgument,
            .ffn_down => {
                if (!self.pending) return error.HipInvalidArgument;
                @memcpy(hidden, self.ffn_out);
                self.pending = false;
            },
            else => return error.HipUnsupportedType,
        }
    }
};

// ---- operator planner (OpScheduler.planLayer with the GPU rules) ----

/// Plans one layer (RMSNorm, attention, RMSNorm, FFN); `out` receives the
/// ops. Returns the number written.
/// A GGUF v3 file mapped and parsed by libmmhip (gguf.loadFromFile,
/// gguf.zig:368-413), for uploading tensors by name.
pub const GgufFile = struct {
    handle: *GgufHandle,

    pub fn open(path: [*:0]const u8) !GgufFile {
        var h: ?*GgufHandle = null;
        try check(mmhip_gguf_open(path, &h));
        return .{ .handle = h.? };
    }

    pub fn close(self: *GgufFile) void {
        mmhip_gguf_close(self.handle);
    }

    pub fn info(self: *const GgufFile) !GgufInfo {
        var i = GgufInfo{};
        try check(mmhip_gguf_get_info(self.handle, &i));
        return i;
    }

    pub fn tensorAt(self: *const GgufFile, index: u64) !GgufTensor {
        var t = GgufTensor{};
        try check(mmhip_gguf_tensor_at(self.handle, index, &t));
        return t;
    }

    pub fn keyAt(self: *const GgufFile, index: u64) ?[*:0]const u8 {
        return mmhip_gguf_key_at(self.handle, index);
    }

    /// tensor_infos.get + tensorPtr (gguf.zig:218-229); null if absent.
    pub fn findTensor(self: *const GgufFile, name: [*:0]const u8) ?GgufTensor {
        var t = GgufTensor{};
        if (mmhip_gguf_find_tensor(self.handle, name, &t) != 0) return null;
        return t;
    }

    /// metaInt / metaFloat / metaString (gguf.zig:232-262); null if absent or of another type.
    pub fn metaInt(self: *const GgufFile, key: [*:0]const u8) ?i64 {
        var v: i64 = 0;
        return if (mmhip_gguf_meta_int(self.handle, key, &v) == 0) v else null;
    }

    pub fn metaFloat(self: *const GgufFile, key: [*:0]const u8) ?f64 {
        var v: f64 = 0;
        return if (mmhip_gguf_meta_float(self.handle, key, &v) == 0) v else null;
    }

    pub fn metaString(self: *const GgufFile, key: [*:0]const u8) ?[]const u8 {
        var p: ?[*]const u8 = null;
        var n: u64 = 0;
        if (mmhip_gguf_meta_string(self.handle, key, &p, &n) != 0) return null;
        return if (n == 0) "" else p.?[0..@intCast(n)];
    }

    /// Metadata value type (MetadataValueType), null if absent.
    pub fn metaType(self: *const GgufFile, key: [*:0]const u8) ?u32 {
        const t = mmhip_gguf_meta_type(self.handle, key);
        return if (t < 0) null else @intCast(t);
    }

    /// Raw array payload: numeric elements little-endian, strings as [u64 len][bytes].
    pub fn metaArray(self: *const GgufFile, key: [*:0]const u8) ?struct { elem_type: u32, len: u64, data: []const u8 } {
        var et: u32 = 0;
        var n: u64 = 0;
        var d: ?*const anyopaque = null;
        var nb: u64 = 0;
        if (mmhip_gguf_meta_array(self.handle, key, &et, &n, &d, &nb) != 0) return null;
        const bytes: []const u8 = if (nb == 0) "" else @as([*]const u8, @ptrCast(d.?))[0..@intCast(nb)];
        return .{ .elem_type = et, .len = n, .data = bytes };
    }

    /// One weight of several matrices' rows stacked in order (same type and
    /// row length), e.g. attn_q_a then attn_kv_a_mqa: one GEMV for both.
    pub fn uploadRows(self: *const GgufFile, backend: *HipBackend, names: []const [*:0]const u8) !*Weight {
        var w: ?*Weight = null;
        try check(mmhip_weight_upload_gguf_rows(backend.ctx, self.handle, names.ptr, @intCast(names.len), &w));
        return w.?;
    }

    /// One-time device upload of a tensor ([cols, rows, count] in ggml order).
    pub fn upload(self: *const GgufFile, backend: *HipBackend, name: [*:0]const u8) !*Weight {
        var w: ?*Weight = null;
        try check(mmhip_weight_upload_gguf(backend.ctx, self.handle, name, &w));
        return w.?;
    }
};

pub fn planLayer(layer: u32, hp: PlanHyperParams, has_gpu: bool, has_npu: bool, throttle_level: i32, db: []const PerfEntry, out: []OpSchedule) !usize {
    var n: usize = 0;
    try check(mmhip_plan_layer(layer, &hp, @intFromBool(has_gpu), @intFromBool(has_npu), throttle_level, if (db.len > 0) db.ptr else null, db.len, out.ptr, out.len, &n));
    return n;
}

pub fn criticalPathUs(ops: []const OpSchedule) u64 {
    return mmhip_plan_critical_path_us(ops.ptr, ops.len);
}

pub fn deviceMask(ops: []const OpSchedule) u8 {
    return @intCast(mmhip_plan_device_mask(ops.ptr, ops.len));
}

test "HipBackend reports availability without crashing" {
    _ = isAvailable();
}
