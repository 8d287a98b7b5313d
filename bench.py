"""Benchmark on one MI355X: quantised GEMV bandwidth (% of HBM peak) and the
MoE FFN layer's µs/token at batch 1 and 64, per workload.

Headline (`value`): IQ2_XXS decode GEMV, GB/s of algorithmic bytes. One step is
the batch-1 GEMV of a GLM-4.7-Flash-shaped layer's routed experts:
  64 expert matrices W[1536 x 2048] with one shared input x[2048], and
  64 expert matrices W[2048 x 1536] with one input per expert,
weights rotating over distinct device copies (> 1 GiB, several times the
256 MiB Infinity Cache), so every step streams its weights from HBM. The step
time and the kernel durations come from the same timed pass: HIP events are
recorded around every launch of it on the library's stream. Every timed pass
(here and in the sections below) follows SETTLE_S seconds of continuous work
on its own calls, then the warm-up calls: from idle, the GPU's clocks and
power take tens of milliseconds of work to settle, and a serving GPU runs
settled. The first 20 headline steps from idle are reported beside the
result (`roofline.settle`).

`configs` holds one object per workload of the path, each with its device
time, GB/s of algorithmic bytes, fraction of the 8 TB/s peak and of the
measured read ceiling, parity against the oracle on the same inputs
(max-abs-rel and the 99.9th percentile of per-element relative error), and
the oracle's CPU time on the box's host cores:
  cfg0  Q8_0 GEMV W[1536 x 2048], batch 1 (matVecMulQ8_0)
  cfg1  IQ2_XXS GEMV W[1536 x 2048] and W[2048 x 1536], batch 1
  cfg2  Q8_0 batched QMM X[64 x 2048] . W[1536 x 2048]^T and
        X[64 x 1536] . W[2048 x 1536]^T (matMulQ8_0 via batchMatMulUnified)
  cfg3  one MoE FFN layer (hidden 2048, 64 IQ2_XXS experts of width 1536,
        top-4 + shared expert, f32 router), batch 1
  cfg4  the same layer on 64 tokens with Zipf(1.1) expert skew (grouped prefill)
Single-matrix workloads rotate over >= 1 GiB of copies (cold), one launch per
call, timed back to back with HIP events (median of blocks).

Also: `stream` (a plain streaming read of 4 GiB: the practical read ceiling),
`q8_gemv` (the headline step with Q8_0 weights), the Q8_0 KV codec, the
output projection + greedy argmax, the MLA projections, and `host` (the
box's CPU model and core count that the CPU baselines ran on).

Flags: --only NAME runs one section (stream, step, cfg0 ... cfg4, q8step, kv,
logits, mla) after a short read-kernel calibration, for the rocprofv3 runs
whose summaries are committed under profiles/; --pmc-summary DIR prints the
per-kernel averages of a rocprofv3 --pmc output directory.
"""
import argparse
import ctypes
import glob
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "mobile-moe.zig_amd")
sys.path.insert(0, os.path.join(PKG, "python"))

import numpy as np  # noqa: E402

import mmhip as mm  # noqa: E402

METRIC = "quant GEMV HBM GB/s (% of peak) + MoE FFN layer µs/token at batch 1 and 64"
HBM_PEAK_GBS = 8000.0
SETTLE_S = 0.25  # seconds of continuous work on a timed pass's own calls before it (HipEvents.settle)
HIDDEN, INTER, EXPERTS = 2048, 1536, 64
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemv_iq2_traffic.txt")
GIB = 1 << 30


class HipEvents:
    """hipEventRecord / hipEventElapsedTime on the library's stream (the stream
    every mmhip launch goes to; torch's events would see only torch's)."""

    def __init__(self):
        self.hip = ctypes.CDLL("libamdhip64.so")
        self.hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.hip.hipStreamSynchronize.argtypes = [ctypes.c_void_p]
        self.pool = []

    def _get(self, n):
        while len(self.pool) < n:
            e = ctypes.c_void_p()
            if self.hip.hipEventCreate(ctypes.byref(e)) != 0:
                raise RuntimeError("hipEventCreate failed")
            self.pool.append(e)
        return self.pool[:n]

    def record(self, e, stream):
        if self.hip.hipEventRecord(e, ctypes.c_void_p(stream)) != 0:
            raise RuntimeError("hipEventRecord failed")

    def elapsed_ms(self, a, b):
        ms = ctypes.c_float()
        if self.hip.hipEventElapsedTime(ctypes.byref(ms), a, b) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return ms.value

    def time_ms(self, stream, fn):
        """Milliseconds of the work `fn` enqueues on `stream`."""
        a, b = self._get(2)
        self.record(a, stream)
        fn()
        self.record(b, stream)
        self.hip.hipEventSynchronize(b)
        return self.elapsed_ms(a, b)

    def settle(self, stream, call, seconds=None):
        """Runs call(i) back to back for `seconds` (SETTLE_S) before a timed
        pass. From idle, the MI355X's clocks and power settle over the first
        tens of milliseconds of continuous work: the headline step measured
        ~23 µs for its first ~60 steps, up to ~32 µs around step 160, and
        ~22.9 µs again after ~800 steps (and at 22.8 µs after 0.3 s of
        work). A serving GPU runs settled, so the timed passes follow this.
        Returns the number of calls made."""
        seconds = SETTLE_S if seconds is None else seconds
        t0 = time.perf_counter()
        i = 0
        while time.perf_counter() - t0 < seconds:
            for _ in range(32):
                call(i)
                i += 1
            self.hip.hipStreamSynchronize(ctypes.c_void_p(stream))
        return i

    def per_call_us(self, stream, call, n_per_block, blocks=5):
        """Median over `blocks` blocks of n back-to-back calls (call(i), i
        running on across blocks), after the GPU has settled on the same
        calls: µs per call."""
        k = [0]
        self.settle(stream, call)

        def block():
            for _ in range(n_per_block):
                call(k[0])
                k[0] += 1

        return float(np.median([self.time_ms(stream, block) / n_per_block for _ in range(blocks)])) * 1e3


# ---------------------------------------------------------------- helpers

def parity(got, ref):
    """max|y - r| / max|r| and the 99.9th percentile of per-element relative
    error |y - r| / max(|r|, 1e-6 max|r|) (the floor keeps near-zero
    references from dominating)."""
    got = np.asarray(got, dtype=np.float64).reshape(-1)
    ref = np.asarray(ref, dtype=np.float64).reshape(-1)
    rel = np.abs(got - ref) / np.maximum(np.abs(ref), 1e-6 * np.max(np.abs(ref)))
    return {"max_abs_rel": float(f"{mm.max_abs_rel(got, ref):.3e}"),
            "p999_rel": float(f"{np.percentile(rel, 99.9):.3e}")}


def rate(nbytes, us, stream_gbs):
    gbs = nbytes / (us * 1e-6) / 1e9
    out = {"us": round(us, 3), "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}
    if stream_gbs:
        out["frac_of_stream"] = round(gbs / stream_gbs, 4)
    return out


def gemv_bytes(fmt, rows, cols, n_mats, shared_x):
    w = mm.tensor_bytes(fmt, rows, cols) * n_mats
    x = cols * 4 * (1 if shared_x else n_mats)
    y = rows * 4 * n_mats
    return w + x + y


def host_info():
    model = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        aff = len(os.sched_getaffinity(0))
    except AttributeError:
        aff = None
    return {"cpu_model": model, "nproc": os.cpu_count(), "cpus_in_affinity": aff}


def oracle():
    """The CPU restatement of the reference, used here only as the parity
    checker and the timed CPU baseline, never inside a GPU timed region."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc
    orc.lib()
    return orc


def cpu_time_us(fn, min_runs=3, max_runs=21, budget_s=2.0):
    """Median µs of fn() after one warm-up call, with at least min_runs runs
    and at most max_runs within about budget_s seconds."""
    fn()
    ts = []
    t_end = time.perf_counter() + budget_s
    while len(ts) < min_runs or (len(ts) < max_runs and time.perf_counter() < t_end):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts)) * 1e6, len(ts)


# ---------------------------------------------------------------- stream

class ReadKernel:
    """The plain streaming-read kernel (lib/libmmbench.so)."""

    def __init__(self, ctx):
        self.ctx = ctx
        self.lib = ctypes.CDLL(os.path.join(PKG, "lib", "libmmbench.so"))
        self.lib.mmbench_read.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p, ctypes.c_uint32,
                                          ctypes.c_void_p]
        self.blocks = 8 * ctx.num_cu
        self.sink = mm.DeviceArray(ctx, 4 * self.blocks)

    def read(self, buf, nbytes):
        if self.lib.mmbench_read(ctypes.c_void_p(buf.ptr), nbytes, ctypes.c_void_p(self.sink.ptr), self.blocks,
                                 ctypes.c_void_p(self.ctx.stream)) != 0:
            raise RuntimeError("mmbench_read failed")

    def free(self):
        self.sink.free()


def stream_section(ctx, ev, gib=4, reps=10):
    rk = ReadKernel(ctx)
    nbytes = gib * GIB
    buf = mm.DeviceArray(ctx, nbytes)
    buf.zero()
    for _ in range(2):
        rk.read(buf, nbytes)
    ctx.synchronize()
    us = ev.per_call_us(ctx.stream, lambda i: rk.read(buf, nbytes), reps, blocks=3)
    buf.free()
    rk.free()
    gbs = nbytes / (us * 1e-6) / 1e9
    return {"read_GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4), "us": round(us, 1),
            "workload": f"plain streaming read of {gib} GiB (short-lived waves, four 16-byte non-temporal loads per thread)"}


def calibration_reads(ctx, n=3, mib=512):
    """Three reads of a known 512 MiB, so a counter run can scale FETCH_SIZE."""
    rk = ReadKernel(ctx)
    buf = mm.DeviceArray(ctx, mib << 20)
    buf.zero()
    for _ in range(n):
        rk.read(buf, mib << 20)
    ctx.synchronize()
    buf.free()
    rk.free()


# ---------------------------------------------------------------- headline step

def step_parity(fmt, raw_gate, raw_down, x_h, xd_h, got_g, got_d, orc):
    """Every matrix of one headline step against the oracle's
    matVecMulUnified on the same inputs: the worst max-abs-rel over the 128
    matrices and the 99.9th percentile of per-element relative error."""
    pg, pd = mm.tensor_bytes(fmt, INTER, HIDDEN), mm.tensor_bytes(fmt, HIDDEN, INTER)
    refs, gots = [], []
    for e in range(EXPERTS):
        refs.append(orc.mat_vec_mul_unified(raw_gate[e * pg:(e + 1) * pg], fmt, x_h, INTER, HIDDEN))
        gots.append(got_g[e])
        refs.append(orc.mat_vec_mul_unified(raw_down[e * pd:(e + 1) * pd], fmt, xd_h[e], HIDDEN, INTER))
        gots.append(got_d[e])
    worst = max(mm.max_abs_rel(gv, rv) for gv, rv in zip(gots, refs))
    p = parity(np.concatenate(gots), np.concatenate(refs))
    return {"max_abs_rel": float(f"{worst:.3e}"), "p999_rel": p["p999_rel"], "matrices": 2 * EXPERTS,
            "checked": "one step's outputs after the timed pass, every matrix against the oracle (bar 1e-3)"}


def step_section(ctx, ev, fmt, steps, warmup, pool_gib, rng, orc=None):
    """64 matrices of each shape per step in ONE launch (mmhip_gemv_grouped_dev:
    gate/up-shaped [1536 x 2048] with a shared x, down-shaped [2048 x 1536] with
    one x each). The timed pass is bracketed by HIP events on the library's
    stream and by host synchronisations: the kernel time per step and the
    wall time per step come from the same pass. For comparison, the two
    shapes as separate launches, timed in blocks of back-to-back launches.
    With the oracle, one step's outputs are then checked matrix by matrix."""
    raw_gate = mm.make_weight(rng, fmt, INTER, HIDDEN, EXPERTS)
    raw_down = mm.make_weight(rng, fmt, HIDDEN, INTER, EXPERTS)
    per_set = mm.tensor_bytes(fmt, INTER, HIDDEN, EXPERTS) + mm.tensor_bytes(fmt, HIDDEN, INTER, EXPERTS)
    n_sets = max(2, int(pool_gib * GIB // per_set))
    sets = [(ctx.upload(raw_gate, fmt, INTER, HIDDEN, EXPERTS), ctx.upload(raw_down, fmt, HIDDEN, INTER, EXPERTS))
            for _ in range(n_sets)]
    if orc is None:
        del raw_gate, raw_down
    x_h = rng.standard_normal(HIDDEN).astype(np.float32)
    xd_h = rng.standard_normal((EXPERTS, INTER)).astype(np.float32)
    x = mm.DeviceArray.from_numpy(ctx, x_h)
    xd = mm.DeviceArray.from_numpy(ctx, xd_h)
    yg = mm.DeviceArray(ctx, EXPERTS * INTER * 4)
    yd = mm.DeviceArray(ctx, EXPERTS * HIDDEN * 4)
    groups = [ctx.gemv_groups([(g, 0, EXPERTS, x, 0, yg, INTER), (d, 0, EXPERTS, xd, INTER, yd, HIDDEN)])
              for g, d in sets]

    def step(i):
        ctx.gemv_grouped_dev(groups[i % n_sets])

    b_gate = gemv_bytes(fmt, INTER, HIDDEN, EXPERTS, True)
    b_down = gemv_bytes(fmt, HIDDEN, INTER, EXPERTS, False)
    st = ctx.stream
    # The first 20 steps from idle (reported, not the result), then the
    # settle phase, the warm-up steps and the timed steps.
    ctx.synchronize()
    first_us = ev.time_ms(st, lambda: [step(i) for i in range(20)]) * 1e3 / 20
    settle_steps = ev.settle(st, step)
    for i in range(warmup):
        step(i)
    ctx.synchronize()
    a, b = ev._get(2)
    t0 = time.perf_counter()
    ev.record(a, st)
    for i in range(steps):
        step(i)
    ev.record(b, st)
    ctx.synchronize()
    dt = time.perf_counter() - t0
    device_us = ev.elapsed_ms(a, b) * 1e3 / steps

    def gate(i):
        ctx.gemv_batched_dev(sets[i % n_sets][0], 0, EXPERTS, x, 0, yg, INTER)

    def down(i):
        ctx.gemv_batched_dev(sets[i % n_sets][1], 0, EXPERTS, xd, INTER, yd, HIDDEN)

    reps = max(10, steps // 4)
    sep = {"gate_1536x2048_us": round(ev.per_call_us(st, gate, reps), 3),
           "down_2048x1536_us": round(ev.per_call_us(st, down, reps), 3)}
    step_par = None
    if orc is not None:
        yg.zero()
        yd.zero()
        step(0)
        ctx.synchronize()
        got_g = yg.to_numpy(np.float32, EXPERTS * INTER).reshape(EXPERTS, INTER)
        got_d = yd.to_numpy(np.float32, EXPERTS * HIDDEN).reshape(EXPERTS, HIDDEN)
        step_par = step_parity(fmt, raw_gate, raw_down, x_h, xd_h, got_g, got_d, orc)
    for g, d in sets:
        g.free()
        d.free()
    for arr in (x, xd, yg, yd):
        arr.free()
    return {"step_bytes": b_gate + b_down, "b_gate": b_gate, "b_down": b_down, "dt": dt, "n_sets": n_sets,
            "pool_gib": n_sets * per_set / GIB, "device_us_per_step": device_us, "separate_launches": sep,
            "first_20_steps_us": first_us, "settle_steps": settle_steps, "parity": step_par}


def read_traffic():
    """HBM bytes (read + written) per launch of the headline step, from the
    committed counter summary (calibrated FETCH_SIZE + WRITE_SIZE)."""
    if not os.path.exists(TRAFFIC_FILE):
        return None
    for line in open(TRAFFIC_FILE):
        if line.split(":")[0].strip() == "hbm_bytes_per_launch":
            return float(line.split(":", 1)[1].split()[0])
    return None


# ---------------------------------------------------------------- configs

def cold_stack(ctx, raw, fmt, rows, cols, pool_gib):
    """One weight of n copies of `raw` (n x [rows x cols], >= pool_gib GiB)."""
    per = mm.tensor_bytes(fmt, rows, cols)
    n = max(2, int(np.ceil(pool_gib * GIB / per)))
    w = ctx.upload(np.tile(raw, n), fmt, rows, cols, n)
    return w, n


def gemv_cfg(ctx, ev, rng, fmt, rows, cols, pool_gib, stream_gbs, orc, reps):
    raw = mm.make_weight(rng, fmt, rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    w, n = cold_stack(ctx, raw, fmt, rows, cols, pool_gib)
    dx = mm.DeviceArray.from_numpy(ctx, x)
    dy = mm.DeviceArray(ctx, rows * 4)
    call = lambda i: ctx.gemv_batched_dev(w, i % n, 1, dx, 0, dy, 0)
    for i in range(8):
        call(i)
    ctx.synchronize()
    us = ev.per_call_us(ctx.stream, call, reps)
    ctx.gemv_batched_dev(w, 0, 1, dx, 0, dy, 0)
    ctx.synchronize()
    got = dy.to_numpy(np.float32, rows)
    for a in (w, dx, dy):
        a.free()
    nbytes = gemv_bytes(fmt, rows, cols, 1, True)
    out = {"shape": f"[{rows} x {cols}]", "bytes": nbytes, **rate(nbytes, us, stream_gbs),
           "copies": n, "pool_MiB": round(n * mm.tensor_bytes(fmt, rows, cols) / (1 << 20))}
    if orc is not None:
        out["parity"] = parity(got, orc.mat_vec_mul_unified(raw, fmt, x, rows, cols))
        cpu_us, runs = cpu_time_us(lambda: orc.mat_vec_mul_unified(raw, fmt, x, rows, cols))
        out["cpu"] = {"us": round(cpu_us, 1), "threads": 1, "runs": runs}
    return out


def qmm_cfg(ctx, ev, rng, rows, cols, batch, pool_gib, stream_gbs, orc, reps):
    fmt = mm.Q8_0
    raw = mm.make_weight(rng, fmt, rows, cols)
    X = rng.standard_normal((batch, cols)).astype(np.float32)
    w, n = cold_stack(ctx, raw, fmt, rows, cols, pool_gib)
    dx = mm.DeviceArray.from_numpy(ctx, X)
    dy = mm.DeviceArray(ctx, batch * rows * 4)
    call = lambda i: ctx.qmm_dev(w, i % n, dx, dy, batch, 0)
    for i in range(8):
        call(i)
    ctx.synchronize()
    us = ev.per_call_us(ctx.stream, call, reps)
    ctx.qmm_dev(w, 0, dx, dy, batch, 0)
    ctx.synchronize()
    got = dy.to_numpy(np.float32, batch * rows).reshape(batch, rows)
    for a in (w, dx, dy):
        a.free()
    nbytes = mm.tensor_bytes(fmt, rows, cols) + X.nbytes + batch * rows * 4
    flop = 2 * batch * rows * cols
    out = {"shape": f"X[{batch} x {cols}] . W[{rows} x {cols}]^T", "bytes": nbytes, **rate(nbytes, us, stream_gbs),
           "TFLOP/s": round(flop / (us * 1e-6) / 1e12, 2), "flop": flop, "copies": n,
           "pool_MiB": round(n * mm.tensor_bytes(fmt, rows, cols) / (1 << 20)),
           "launches_per_call": 1 if cols <= 2048 else 2,
           "note": ("one launch per call: the activations are quantised inside the int8-digit MFMA kernel"
                    if cols <= 2048 else "two launches per call: activation quantisation, then the int8-digit MFMA")}
    if orc is not None:
        ref = orc.batch_mat_mul_unified(raw, fmt, X, rows, batch, cols).reshape(batch, rows)
        out["parity"] = parity(got, ref)
        cpu_us, runs = cpu_time_us(lambda: orc.batch_mat_mul_unified(raw, fmt, X, rows, batch, cols),
                                   min_runs=2, max_runs=5, budget_s=3.0)
        out["cpu"] = {"us": round(cpu_us, 1), "threads": 1, "runs": runs}
    return out


def moe_weights(rng):
    gate = mm.make_iq2_xxs(rng, INTER, HIDDEN, EXPERTS)
    up = mm.make_iq2_xxs(rng, INTER, HIDDEN, EXPERTS)
    down = mm.make_iq2_xxs(rng, HIDDEN, INTER, EXPERTS)
    shared = (mm.make_iq2_xxs(rng, INTER, HIDDEN), mm.make_iq2_xxs(rng, INTER, HIDDEN),
              mm.make_iq2_xxs(rng, HIDDEN, INTER))
    router = rng.normal(0.0, 0.02, (EXPERTS, HIDDEN)).astype(np.float32)
    return router, gate, up, down, shared


def zipf_batch(rng, t, s=1.1):
    """Hidden states for the grouped prefill case: under an identity router the
    first 64 coordinates are the logits, N(0, 1) plus 10 on 4 experts per token
    drawn without replacement from Zipf(s) over a seeded expert permutation."""
    perm = rng.permutation(EXPERTS)
    p = 1.0 / np.arange(1, EXPERTS + 1) ** s
    p /= p.sum()
    h = rng.standard_normal((t, HIDDEN)).astype(np.float32)
    for ti in range(t):
        h[ti, perm[rng.choice(EXPERTS, 4, replace=False, p=p)]] += 10.0
    router = np.zeros((EXPERTS, HIDDEN), dtype=np.float32)
    router[:, :EXPERTS] = np.eye(EXPERTS, dtype=np.float32)
    return h, router


def moe_section(ctx, ev, rng, calls, stream_gbs, orc, n_layers=8, n_tokens=61, which=(1, 64)):
    """MoE layer µs/token. Cold: calls rotate over n_layers layers (each with its
    own 64 experts, 158 MB) and, at batch 1, over n_tokens distinct tokens, so
    the routed experts change from call to call and the touched weights
    (about 0.6 GB at batch 1, 1 GB at batch 64) exceed the 256 MB
    Infinity Cache. Warm: one layer and one input repeated."""
    router, gate, up, down, shared = moe_weights(rng)
    h64, id_router = zipf_batch(rng, 64)
    kw = dict(hidden=HIDDEN, inter=INTER, n_experts=EXPERTS, expert_type=mm.IQ2_XXS, gate=gate, up=up, down=down,
              shared=shared, shared_inter=INTER)
    toks = rng.standard_normal((n_tokens, HIDDEN)).astype(np.float32)
    stream = ctx.stream
    res = {}
    expert_bytes = 3 * mm.tensor_bytes(mm.IQ2_XXS, INTER, HIDDEN)
    router_bytes = EXPERTS * HIDDEN * 4
    for t in which:
        rt = router if t == 1 else id_router
        layers = [mm.MoeLayer(ctx, router=rt, **kw) for _ in range(n_layers)]
        hs = ([mm.DeviceArray.from_numpy(ctx, toks[j:j + 1]) for j in range(n_tokens)] if t == 1
              else [mm.DeviceArray.from_numpy(ctx, h64)])
        od = mm.DeviceArray(ctx, t * HIDDEN * 4)
        n = calls if t == 1 else max(10, calls // 4)
        n = max(n, 2 * n_layers)

        def run(i):
            layers[i % n_layers].ffn_dev(hs[i % len(hs)], od, t)

        ev.settle(stream, run)
        for i in range(2 * n_layers):
            run(i)
        ctx.synchronize()
        cold = ev.time_ms(stream, lambda: [run(i) for i in range(n)]) / n * 1e3 / t
        ev.settle(stream, lambda i: layers[0].ffn_dev(hs[0], od, t))
        for _ in range(5):
            layers[0].ffn_dev(hs[0], od, t)
        ctx.synchronize()
        warm = ev.time_ms(stream, lambda: [layers[0].ffn_dev(hs[0], od, t) for _ in range(n)]) / n * 1e3 / t
        if t == 1:
            touched = 4
            nbytes = router_bytes + 5 * expert_bytes + 2 * HIDDEN * 4
            h_in = toks[:1]
        else:
            touched = len(set(np.argsort(-h64[:, :EXPERTS], axis=1)[:, :4].reshape(-1).tolist()))
            nbytes = (touched + 1) * expert_bytes + router_bytes + 2 * t * HIDDEN * 4
            h_in = h64
        out_g, ids_g, w_g = layers[0].ffn(h_in)
        for h in hs:
            h.free()
        od.free()
        for layer in layers:
            layer.free()
        r = {"us_per_token": round(cold, 3), "us_per_token_warm": round(warm, 3), "tokens": t,
             "us_per_call": round(cold * t, 2), "bytes_per_call": nbytes,
             **{k: v for k, v in rate(nbytes, cold * t, stream_gbs).items() if k != "us"},
             "experts_touched": touched}
        if orc is not None:
            cpu = orc.Moe(router=rt, **{**kw, "expert_type": orc.IQ2_XXS})
            pool = orc.Pool(4)
            try:
                out_c, ids_c, w_c = cpu.ffn(h_in, pool=pool)
            finally:
                pool.close()
            r["parity"] = parity(out_g, out_c)
            r["parity"]["route_ids_equal"] = bool(np.array_equal(ids_g, ids_c))
            r["parity"]["route_weights_max_rel"] = float(f"{np.max(np.abs(w_g - w_c) / np.maximum(np.abs(w_c), 1e-30)):.3e}")
        res[t] = r
    return res, (router, gate, up, down, shared, h64, id_router)


def cpu_moe_baseline(weights, tokens):
    """Oracle moeFFN with the reference's 4-worker pool (5 threads with the
    caller), one call per token as forwardBatch does."""
    orc = oracle()
    router, gate, up, down, shared, h64, id_router = weights
    kw = dict(hidden=HIDDEN, inter=INTER, n_experts=EXPERTS, expert_type=orc.IQ2_XXS, gate=gate, up=up, down=down,
              shared=shared, shared_inter=INTER)
    pool = orc.Pool(4)
    try:
        moe = orc.Moe(router=router, **kw)
        h1 = np.random.default_rng(7).standard_normal((1, HIDDEN)).astype(np.float32)
        b1, runs = cpu_time_us(lambda: moe.ffn(h1, pool=pool), min_runs=3, max_runs=7, budget_s=3.0)
        moe64 = orc.Moe(router=id_router, **kw)
        t0 = time.perf_counter()
        moe64.ffn(h64[:tokens], pool=pool)
        b64 = (time.perf_counter() - t0) / tokens
    finally:
        pool.close()
    return {"batch1_us_per_token": round(b1, 1), "batch64_us_per_token": round(b64 * 1e6, 1),
            "unit": "µs/token", "cores": 5, "kind": "port",
            "sample": f"median of {runs} batch-1 calls; the first {tokens} tokens of the batch-64 case, "
                      f"one moeFFN per token"}


def cpu_gemv_baseline(seconds):
    """Oracle IQ2_XXS GEMV (dequantize + f32 GEMV, one thread), bounded sample:
    alternating [1536 x 2048] and [2048 x 1536] matrices for about `seconds`."""
    orc = oracle()
    rng = np.random.default_rng(99)
    mats = [(mm.make_iq2_xxs(rng, INTER, HIDDEN), INTER, HIDDEN), (mm.make_iq2_xxs(rng, HIDDEN, INTER), HIDDEN, INTER)]
    xs = [rng.standard_normal(HIDDEN).astype(np.float32), rng.standard_normal(INTER).astype(np.float32)]
    n = nbytes = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        raw, r, c = mats[n % 2]
        orc.mat_vec_mul_unified(raw, orc.IQ2_XXS, xs[n % 2], r, c)
        nbytes += gemv_bytes(mm.IQ2_XXS, r, c, 1, True)
        n += 1
    dt = time.perf_counter() - t0
    return {"value": round(nbytes / dt / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{n} IQ2_XXS GEMVs alternating [1536x2048]/[2048x1536] in {dt:.1f} s, "
                      f"{dt / n * 1e6:.0f} us per GEMV (dequantize to f32, then the 4-lane f32 GEMV)"}


# ---------------------------------------------------------------- other rows of the path

def kv_codec_section(ctx, ev, rng, reps=20, n_rows=131072, row_len=576):
    """Q8_0 KV-cache codec (KVCache.put / getKVCompressed's Q8_0 branches,
    kv_cache.zig:225-349): n_rows positions x row_len values (kv_lora_rank 512
    + rope dim 64) quantised to 34-byte blocks and dequantised back; rates
    in algorithmic bytes (f32 in / out, 34 B per 32 values) per kernel."""
    x = rng.standard_normal((n_rows, row_len)).astype(np.float32)
    nbytes = n_rows * ((row_len + 31) // 32) * 34
    dx = mm.DeviceArray.from_numpy(ctx, x)
    db = mm.DeviceArray(ctx, nbytes)
    dy = mm.DeviceArray(ctx, x.nbytes)
    st = ctx.stream
    q = lambda: ctx.quantize_q8_0_rows_dev(db, dx, row_len, n_rows, row_len)
    d = lambda: ctx.dequantize_q8_0_rows_dev(dy, row_len, db, n_rows, row_len)
    for _ in range(3):
        q()
        d()
    ctx.synchronize()
    out = {}
    for name, fn in (("quantize", q), ("dequantize", d)):
        us = ev.per_call_us(st, lambda i: fn(), reps)
        gbs = (x.nbytes + nbytes) / (us * 1e-6) / 1e9
        out[name] = {"us": round(us, 2), "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}
    for a in (dx, db, dy):
        a.free()
    out["workload"] = (f"{n_rows} positions x {row_len} f32 (kv_lora 512 + rope 64) <-> Q8_0 blocks; "
                       f"{x.nbytes + nbytes} algorithmic bytes per kernel call")
    return out


def dequant_section(ctx, ev, rng, orc, reps=20, n_mats=16):
    """dequantize (dequant.zig:632-659) of raw GGUF blocks on the device:
    n_mats expert matrices [1536 x 2048] of Q8_0 (dequantizeQ8_0Slice,
    133-142) and of IQ2_XXS (dequantizeIQ2XXS, 358-369) to f32 in one call
    each; rates in algorithmic bytes (raw blocks in, f32 out). The CPU line is
    the oracle's dequantize of one such matrix on one core (the reference
    dequantizes the whole f32 matrix before each IQ2_XXS GEMV)."""
    out = {"workload": f"{n_mats} x [{INTER} x {HIDDEN}] raw GGUF blocks -> f32, one call per type"}
    st = ctx.stream
    n = n_mats * INTER * HIDDEN
    od = mm.DeviceArray(ctx, n * 4)
    for name, fmt in (("q8_0", mm.Q8_0), ("iq2_xxs", mm.IQ2_XXS)):
        raw = mm.make_weight(rng, fmt, INTER, HIDDEN, n_mats)
        rd = mm.DeviceArray.from_numpy(ctx, raw)
        for _ in range(3):
            ctx.dequantize_dev(od, rd, fmt, n)
        ctx.synchronize()
        us = ev.per_call_us(st, lambda i: ctx.dequantize_dev(od, rd, fmt, n), reps)
        nbytes = raw.nbytes + n * 4
        gbs = nbytes / (us * 1e-6) / 1e9
        r = {"us": round(us, 2), "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4), "bytes": nbytes}
        if orc is not None:
            one = raw[: raw.nbytes // n_mats]
            m = INTER * HIDDEN
            ref = orc.dequantize(one, fmt, m)
            got = od.to_numpy(np.float32, m)
            r["bit_exact_first_matrix"] = bool(np.array_equal(got.view(np.uint32), ref.view(np.uint32)))
            cus, runs = cpu_time_us(lambda: orc.dequantize(one, fmt, m))
            r["cpu"] = {"us_per_matrix": round(cus, 1), "threads": 1, "runs": runs}
        rd.free()
        out[name] = r
    od.free()
    return out


def cpu_kv_codec_baseline(rng, seconds=2.0, row_len=576):
    """Oracle quantizeQ8_0 per row on one core (KVCache.put's loop), bounded sample."""
    orc = oracle()
    x = rng.standard_normal((4096, row_len)).astype(np.float32)
    nbytes = x.nbytes + 4096 * ((row_len + 31) // 32) * 34
    n = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        orc.quantize_q8_0_rows(x, row_len)
        n += 1
    dt = time.perf_counter() - t0
    return {"value": round(nbytes * n / dt / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{n} x quantise 4096 positions x {row_len} values in {dt:.1f} s"}


def logits_section(ctx, ev, rng, pool_gib, reps=20, vocab=154880, hidden=HIDDEN):
    """computeLogits + sampleGreedy (inference.zig:1189-1197, 376-386): the
    output projection GEMV [vocab x hidden] in Q8_0 and IQ2_XXS (the GGUF's
    type decides), weights rotating over >= pool_gib GiB of copies, then the
    greedy argmax over the logits on the device."""
    x = mm.DeviceArray.from_numpy(ctx, rng.standard_normal(hidden).astype(np.float32))
    y = mm.DeviceArray(ctx, vocab * 4)
    tok = mm.DeviceArray(ctx, 4)
    st = ctx.stream
    out = {"workload": f"output projection [{vocab} x {hidden}] GEMV + greedy argmax over {vocab} logits"}
    for name, t in (("q8_0", mm.Q8_0), ("iq2_xxs", mm.IQ2_XXS)):
        raw = mm.make_weight(rng, t, vocab, hidden)
        n_sets = max(3, int(np.ceil(pool_gib * GIB / raw.nbytes)))
        ws = [ctx.upload(raw, t, vocab, hidden) for _ in range(n_sets)]
        call = lambda i: ctx.gemv_batched_dev(ws[i % n_sets], 0, 1, x, 0, y, 0)
        for i in range(2 * n_sets):
            call(i)
        ctx.synchronize()
        us = ev.per_call_us(st, call, reps)
        nbytes = raw.nbytes + hidden * 4 + vocab * 4
        out[name] = {"us": round(us, 2), "GB/s": round(nbytes / (us * 1e-6) / 1e9, 1),
                     "frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4), "weight_bytes": int(raw.nbytes),
                     "copies": n_sets, "pool_MiB": round(n_sets * raw.nbytes / (1 << 20))}
        for w in ws:
            w.free()
    for _ in range(3):
        ctx.argmax_dev(tok, y, vocab)
    ctx.synchronize()
    out["argmax_us"] = round(ev.per_call_us(st, lambda i: ctx.argmax_dev(tok, y, vocab), reps), 2)
    for a in (x, y, tok):
        a.free()
    return out


def mla_section(ctx, ev, rng, pool_gib, reps=20, batch=64):
    """MLA attention projections (inference.zig:467-489, 663-665; batch path
    684-706, 880-882) on the same kernels: q_a [768 x 2048], q_b [3840 x 768],
    kv_a [576 x 2048], o_proj [2048 x 2560], one layer's four GEMVs per decode
    step with the weights of as many layers as fill >= pool_gib GiB rotating
    (cold, as in decode), and the four batched products at 64 tokens."""
    shapes = {"q_a": (768, 2048), "q_b": (3840, 768), "kv_a": (576, 2048), "o_proj": (2048, 2560)}
    st = ctx.stream
    xs = {n: mm.DeviceArray.from_numpy(ctx, rng.standard_normal(batch * c).astype(np.float32))
          for n, (_, c) in shapes.items()}
    ys = {n: mm.DeviceArray(ctx, batch * r * 4) for n, (r, _) in shapes.items()}
    ys["qkv_a"] = mm.DeviceArray(ctx, (768 + 576) * 4)
    out = {"workload": "MLA projections: " + ", ".join(f"{n} [{r}x{c}]" for n, (r, c) in shapes.items()) +
                       "; decode = the four GEMVs of one layer (fused: q_a and kv_a as one stacked weight), "
                       f"batch = the four products at {batch} tokens"}
    for name, t in (("q8_0", mm.Q8_0), ("iq2_xxs", mm.IQ2_XXS)):
        raws = {n: mm.make_weight(rng, t, r, c) for n, (r, c) in shapes.items()}
        wbytes = sum(int(r.nbytes) for r in raws.values())
        n_layers = max(47, int(np.ceil(pool_gib * GIB / wbytes)))
        layers = [{n: ctx.upload(raws[n], t, r, c) for n, (r, c) in shapes.items()} for _ in range(n_layers)]
        qkv = np.concatenate([raws["q_a"], raws["kv_a"]])
        fused = [ctx.upload(qkv, t, 768 + 576, 2048) for _ in range(n_layers)]

        def decode(i):
            lw = layers[i % n_layers]
            for n in shapes:
                ctx.gemv_batched_dev(lw[n], 0, 1, xs[n], 0, ys[n], 0)

        def prefill(i):
            lw = layers[i % n_layers]
            for n in shapes:
                ctx.qmm_dev(lw[n], 0, xs[n], ys[n], batch)

        # q_a and kv_a read the same hidden vector: one weight of 768 + 576
        # stacked rows (the raw rows concatenated), so three launches per layer.
        def decode_fused(i):
            lw = layers[i % n_layers]
            ctx.gemv_batched_dev(fused[i % n_layers], 0, 1, xs["q_a"], 0, ys["qkv_a"], 0)
            for n in ("q_b", "o_proj"):
                ctx.gemv_batched_dev(lw[n], 0, 1, xs[n], 0, ys[n], 0)

        res = {}
        for label, fn in (("decode", decode), ("decode_fused_qkv_a", decode_fused), ("batch64", prefill)):
            for i in range(n_layers):
                fn(i)
            ctx.synchronize()
            res[label + "_us_per_layer"] = round(ev.per_call_us(st, fn, reps), 2)
        nbytes = wbytes + sum(4 * (r + c) for r, c in shapes.values())
        res["decode_GB/s"] = round(nbytes / (res["decode_us_per_layer"] * 1e-6) / 1e9, 1)
        res["decode_frac"] = round(res["decode_GB/s"] / HBM_PEAK_GBS, 4)
        res["weight_bytes_per_layer"] = wbytes
        res["layers_rotating"] = n_layers
        res["pool_MiB"] = round(n_layers * (wbytes + int(qkv.nbytes)) / (1 << 20))
        out[name] = res
        for lw in layers:
            for w in lw.values():
                w.free()
        for w in fused:
            w.free()
    for a in list(xs.values()) + list(ys.values()):
        a.free()
    return out


# ---------------------------------------------------------------- counter summaries

def pmc_summary(path):
    """Per-kernel means of every counter in a rocprofv3 --pmc output directory
    (its *counter_collection.csv), plus the FETCH_SIZE / WRITE_SIZE scale
    from the read kernel of known size (512 MiB per dispatch) when present."""
    import csv
    files = glob.glob(os.path.join(path, "**", "*counter_collection.csv"), recursive=True)
    if not files:
        print(f"no counter_collection.csv under {path}")
        return
    acc = {}
    for f in files:
        for row in csv.DictReader(open(f)):
            name = row.get("Kernel_Name", "?")
            key = (name, row.get("Counter_Name"))
            did = row.get("Dispatch_Id") or row.get("Correlation_Id")
            d = acc.setdefault(key, {})
            d[did] = d.get(did, 0.0) + float(row.get("Counter_Value", 0.0))
    kernels = {}
    for (name, counter), per in acc.items():
        kernels.setdefault(name, {})[counter] = (float(np.mean(list(per.values()))), len(per))
    scale = {}
    for name, cs in kernels.items():
        if "read_kernel" in name:
            for c in ("FETCH_SIZE",):
                if c in cs and cs[c][0] > 0:
                    scale[c] = (512 << 20) / (cs[c][0] * 1024)
    for name in sorted(kernels):
        short = name if len(name) < 110 else name[:107] + "..."
        print(short)
        for c, (v, n) in sorted(kernels[name].items()):
            line = f"    {c:32s} mean {v:16.1f} over {n} dispatches"
            if c in ("FETCH_SIZE", "WRITE_SIZE"):
                line += f"   = {v * 1024:14.0f} B raw"
                if c in scale:
                    line += f"   x {scale[c]:.3f} = {v * 1024 * scale[c]:14.0f} B"
            print(line)
    if scale:
        print("scale from read_kernel (512 MiB known):", {k: round(v, 4) for k, v in scale.items()})


# ---------------------------------------------------------------- main

def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--pool-gib", type=float, default=1.25)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--cpu-moe-tokens", type=int, default=8)
    ap.add_argument("--no-cpu", action="store_true", help="skip the oracle (parity and CPU baselines)")
    ap.add_argument("--only", default=None,
                    help="run one section: stream, step, cfg0, cfg1, cfg2, cfg3, cfg4, q8step, kv, dequant, logits, mla")
    ap.add_argument("--pmc-summary", default=None, metavar="DIR",
                    help="summarise a rocprofv3 --pmc output directory and exit")
    args = ap.parse_args()
    if args.pmc_summary:
        pmc_summary(args.pmc_summary)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); "
              "this build has no multi-GPU path", file=sys.stderr)
        sys.exit(2)

    ctx = mm.Context(0)
    ev = HipEvents()
    rng = np.random.default_rng(1234)
    orc = None if args.no_cpu else oracle()
    only = args.only
    reps = max(10, args.steps // 4)

    if only:
        calibration_reads(ctx)
        res = {}
        if only == "stream":
            res = stream_section(ctx, ev)
        elif only in ("step", "q8step"):
            fmt = mm.IQ2_XXS if only == "step" else mm.Q8_0
            g = step_section(ctx, ev, fmt, args.steps, args.warmup, args.pool_gib, rng, orc)
            res = {k: (round(v, 3) if isinstance(v, float) else v) for k, v in g.items()}
        elif only == "cfg0":
            res = gemv_cfg(ctx, ev, rng, mm.Q8_0, INTER, HIDDEN, args.pool_gib, None, orc, reps)
        elif only == "cfg1":
            res = {"a": gemv_cfg(ctx, ev, rng, mm.IQ2_XXS, INTER, HIDDEN, args.pool_gib, None, orc, reps),
                   "b": gemv_cfg(ctx, ev, rng, mm.IQ2_XXS, HIDDEN, INTER, args.pool_gib, None, orc, reps)}
        elif only == "cfg2":
            res = {"a": qmm_cfg(ctx, ev, rng, INTER, HIDDEN, 64, args.pool_gib, None, orc, reps),
                   "b": qmm_cfg(ctx, ev, rng, HIDDEN, INTER, 64, args.pool_gib, None, orc, reps)}
        elif only in ("cfg3", "cfg4"):
            res = moe_section(ctx, ev, rng, max(50, args.steps), None, orc, which=(1,) if only == "cfg3" else (64,))[0]
        elif only == "kv":
            res = kv_codec_section(ctx, ev, rng)
        elif only == "dequant":
            res = dequant_section(ctx, ev, rng, orc)
        elif only == "logits":
            res = logits_section(ctx, ev, rng, args.pool_gib)
        elif only == "mla":
            res = mla_section(ctx, ev, rng, args.pool_gib)
        else:
            raise SystemExit(f"unknown section {only}")
        ctx.close()
        print(json.dumps({"only": only, "result": res}), flush=True)
        return

    stream = stream_section(ctx, ev)
    sgbs = stream["read_GB/s"]
    g = step_section(ctx, ev, mm.IQ2_XXS, args.steps, args.warmup, args.pool_gib, rng, orc)
    value = g["step_bytes"] * args.steps / g["dt"] / 1e9
    kernel_us = g["device_us_per_step"]
    achieved = g["step_bytes"] / (kernel_us * 1e-6) / 1e9
    traffic = read_traffic()
    q8 = step_section(ctx, ev, mm.Q8_0, max(20, args.steps // 4), max(5, args.warmup // 4), args.pool_gib, rng,
                      orc)
    q8_steps = max(20, args.steps // 4)

    configs = {
        "cfg0": {"workload": "Q8_0 matVecMul, single token: W[1536 x 2048], x ~ N(0,1)",
                 **gemv_cfg(ctx, ev, rng, mm.Q8_0, INTER, HIDDEN, args.pool_gib, sgbs, orc, reps)},
        "cfg1a": {"workload": "IQ2_XXS GEMV, decode: W[1536 x 2048], batch 1",
                  **gemv_cfg(ctx, ev, rng, mm.IQ2_XXS, INTER, HIDDEN, args.pool_gib, sgbs, orc, reps)},
        "cfg1b": {"workload": "IQ2_XXS GEMV, decode: W[2048 x 1536], batch 1",
                  **gemv_cfg(ctx, ev, rng, mm.IQ2_XXS, HIDDEN, INTER, args.pool_gib, sgbs, orc, reps)},
        "cfg2a": {"workload": "Q8_0 batched QMM, gate/up: X[64 x 2048] -> [64 x 1536]",
                  **qmm_cfg(ctx, ev, rng, INTER, HIDDEN, 64, args.pool_gib, sgbs, orc, reps)},
        "cfg2b": {"workload": "Q8_0 batched QMM, down: X[64 x 1536] -> [64 x 2048]",
                  **qmm_cfg(ctx, ev, rng, HIDDEN, INTER, 64, args.pool_gib, sgbs, orc, reps)},
    }
    moe, weights = moe_section(ctx, ev, rng, max(50, args.steps), sgbs, orc)
    configs["cfg3"] = {"workload": "one MoE FFN layer, GLM-4.7-Flash shape (hidden 2048, 64 IQ2_XXS experts of "
                                   "width 1536, top-4 + shared, f32 router), batch 1; cold: eight layers and 61 "
                                   "tokens rotate; warm: one layer, one token", **moe[1]}
    configs["cfg4"] = {"workload": "grouped-expert MoE prefill: 64 tokens, top-4 over 64 IQ2_XXS experts with "
                                   "Zipf(1.1) skew (identity router on +10 logits), shared expert, scatter-add; "
                                   "cold: eight layers rotate", **moe[64]}

    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(g["dt"] / args.steps * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "iq2_xxs weights x int16 block fixed-point activations (two int8 digits), int32 MFMA, f32 scale",
        "data": "synthetic",
        "config": {
            "workload": "IQ2_XXS decode GEMV, batch 1: 64 expert matrices [1536x2048] (shared x) + "
                        "64 expert matrices [2048x1536] (one x each) per step, both shapes in one launch, "
                        f"weights rotating over {g['n_sets']} distinct copies ({g['pool_gib']:.2f} GiB)",
            "hidden": HIDDEN, "expert_inter": INTER, "experts_per_launch": EXPERTS,
            "bytes_per_step": g["step_bytes"],
        },
        "parity": g["parity"],
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None if traffic is None else round(traffic),
            "kernel": "gemv_iq2_kernel, both shapes in one launch (mmhip_gemv_grouped_dev)",
            "kernel_us_per_step": round(kernel_us, 3),
            "bytes_per_step": g["step_bytes"],
            "frac_of_stream": round(achieved / sgbs, 4),
            "timing": "HIP events around the timed pass of ms_per_step (back-to-back launches, one per step)",
            "settle": {"seconds": SETTLE_S, "steps": g["settle_steps"],
                       "first_20_steps_us": round(g["first_20_steps_us"], 3),
                       "note": "the timed pass follows the settle steps and the warm-up steps; the first 20 steps "
                               "from idle run while the GPU's clocks and power settle (not the result)"},
            "separate_launches": g["separate_launches"],
        },
        "stream": stream,
        "configs": configs,
        "q8_gemv": {"value": round(q8["step_bytes"] * q8_steps / q8["dt"] / 1e9, 2), "unit": "GB/s",
                    "kernel_us_per_step": round(q8["device_us_per_step"], 3),
                    "achieved": round(q8["step_bytes"] / (q8["device_us_per_step"] * 1e-6) / 1e9, 1),
                    "frac": round(q8["step_bytes"] / (q8["device_us_per_step"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                    "separate_launches": q8["separate_launches"],
                    "parity": q8["parity"],
                    "workload": "the headline step with Q8_0 weights (64 + 64 matrices, one launch)"},
        "host": host_info(),
    }
    out["kv_q8_codec"] = kv_codec_section(ctx, ev, rng)
    out["dequantize"] = dequant_section(ctx, ev, rng, orc)
    out["logits"] = logits_section(ctx, ev, rng, args.pool_gib)
    out["mla"] = mla_section(ctx, ev, rng, args.pool_gib)
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_gemv_baseline(args.cpu_seconds)
        out["cpu_baseline"]["host"] = out["host"]
        out["kv_q8_codec"]["cpu_quantize"] = cpu_kv_codec_baseline(rng)
        out["cpu_moe"] = cpu_moe_baseline(weights, args.cpu_moe_tokens)
        out["cpu_moe"]["host"] = out["host"]
    ctx.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
