"""Benchmark on one MI355X: IQ2_XXS decode GEMV bandwidth and the MoE FFN
layer's µs/token at batch 1 and 64.

Headline (`value`): IQ2_XXS decode GEMV, GB/s of algorithmic bytes. One step is
the batch-1 GEMV of a GLM-4.7-Flash-shaped layer's routed experts:
  launch 1: 64 expert matrices W[1536 x 2048], one shared input x[2048]
  launch 2: 64 expert matrices W[2048 x 1536], one input per expert
Weights rotate over distinct device copies (> 1 GiB, several times the
256 MiB Infinity Cache), so every step streams its weights from HBM.

Also reported:
  roofline      the GEMV kernel: algorithmic bytes per launch / its duration,
                the median over alternating blocks of back-to-back launches
                of each shape (HIP event pairs on the library's stream), against the
                8 TB/s HBM peak; `traffic` is the HBM bytes per launch from the
                FETCH_SIZE / WRITE_SIZE counter runs summarised in
                profiles/gemv_iq2_traffic.txt (null when that file is absent)
  moe           one MoE FFN layer (hidden 2048, 64 IQ2_XXS experts of width
                1536, top-4 + shared expert, f32 router): device time per call
                / tokens at batch 1 and batch 64, weights cold (four layers
                rotate); batch 64 routes with Zipf(1.1) skew through an
                identity router, as the grouped prefill case prescribes
  q8_gemv       the same GEMV step with Q8_0 weights (GB/s)
  cpu_baseline  the oracle's CPU path (reference algorithm: dequantize, then
                the 4-lane f32 GEMV) on one host core, bounded sample
  cpu_moe       the oracle's moeFFN with the reference's 4-worker pool
"""
import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "mobile-moe.zig_amd", "python"))

import numpy as np  # noqa: E402

import mmhip as mm  # noqa: E402

METRIC = "quant GEMV HBM GB/s (% of peak) + MoE FFN layer µs/token at batch 1 and 64"
HBM_PEAK_GBS = 8000.0
HIDDEN, INTER, EXPERTS = 2048, 1536, 64
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemv_iq2_traffic.txt")


class HipEvents:
    """hipEventRecord / hipEventElapsedTime on an existing stream."""

    def __init__(self):
        self.hip = ctypes.CDLL("libamdhip64.so")
        self.hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventDestroy.argtypes = [ctypes.c_void_p]

    def time_ms(self, stream, fn):
        """Milliseconds of the work `fn` enqueues on `stream`."""
        a, b = ctypes.c_void_p(), ctypes.c_void_p()
        for e in (a, b):
            if self.hip.hipEventCreate(ctypes.byref(e)) != 0:
                raise RuntimeError("hipEventCreate failed")
        self.hip.hipEventRecord(a, ctypes.c_void_p(stream))
        fn()
        self.hip.hipEventRecord(b, ctypes.c_void_p(stream))
        self.hip.hipEventSynchronize(b)
        ms = ctypes.c_float()
        self.hip.hipEventElapsedTime(ctypes.byref(ms), a, b)
        self.hip.hipEventDestroy(a)
        self.hip.hipEventDestroy(b)
        return ms.value


def gemv_bytes(fmt, rows, cols, n_mats, shared_x):
    w = mm.tensor_bytes(fmt, rows, cols) * n_mats
    x = cols * 4 * (1 if shared_x else n_mats)
    y = rows * 4 * n_mats
    return w + x + y


def read_traffic():
    """HBM bytes per launch of each GEMV shape, from the committed summary."""
    if not os.path.exists(TRAFFIC_FILE):
        return None
    vals = {}
    for line in open(TRAFFIC_FILE):
        if ":" in line and line.split(":")[0].strip() in ("gate_bytes_per_launch", "down_bytes_per_launch"):
            k, v = line.split(":", 1)
            vals[k.strip()] = float(v.split()[0])
    if len(vals) != 2:
        return None
    return vals


def gemv_section(ctx, ev, fmt, steps, warmup, pool_gib, rng):
    raw_gate = mm.make_weight(rng, fmt, INTER, HIDDEN, EXPERTS)
    raw_down = mm.make_weight(rng, fmt, HIDDEN, INTER, EXPERTS)
    per_set = mm.tensor_bytes(fmt, INTER, HIDDEN, EXPERTS) + mm.tensor_bytes(fmt, HIDDEN, INTER, EXPERTS)
    n_sets = max(2, int(pool_gib * (1 << 30) // per_set))
    sets = [(ctx.upload(raw_gate, fmt, INTER, HIDDEN, EXPERTS), ctx.upload(raw_down, fmt, HIDDEN, INTER, EXPERTS))
            for _ in range(n_sets)]
    del raw_gate, raw_down
    x = mm.DeviceArray.from_numpy(ctx, rng.standard_normal(HIDDEN).astype(np.float32))
    xd = mm.DeviceArray.from_numpy(ctx, rng.standard_normal((EXPERTS, INTER)).astype(np.float32))
    yg = mm.DeviceArray(ctx, EXPERTS * INTER * 4)
    yd = mm.DeviceArray(ctx, EXPERTS * HIDDEN * 4)

    def gate(i):
        ctx.gemv_batched_dev(sets[i % n_sets][0], 0, EXPERTS, x, 0, yg, INTER)

    def down(i):
        ctx.gemv_batched_dev(sets[i % n_sets][1], 0, EXPERTS, xd, INTER, yd, HIDDEN)

    b_gate = gemv_bytes(fmt, INTER, HIDDEN, EXPERTS, True)
    b_down = gemv_bytes(fmt, HIDDEN, INTER, EXPERTS, False)
    for i in range(warmup):
        gate(i)
        down(i)
    ctx.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        gate(i)
        down(i)
    ctx.synchronize()
    dt = time.perf_counter() - t0
    # Kernel durations: event pairs around blocks of back-to-back launches of
    # one shape, the shapes' blocks alternating; the median block gives the
    # per-launch time (the device's clock state drifts over a long run, and a
    # single block can land in a slow stretch).
    stream = ctx.stream
    blocks, per = 7, max(10, steps // 4)
    g_blk, d_blk = [], []
    for b in range(blocks):
        g_blk.append(ev.time_ms(stream, lambda: [gate(b * per + i) for i in range(per)]) / per)
        d_blk.append(ev.time_ms(stream, lambda: [down(b * per + i) for i in range(per)]) / per)
    g_ms, d_ms = float(np.median(g_blk)), float(np.median(d_blk))
    for g, d in sets:
        g.free()
        d.free()
    for a in (x, xd, yg, yd):
        a.free()
    return {"step_bytes": b_gate + b_down, "b_gate": b_gate, "b_down": b_down, "dt": dt, "n_sets": n_sets,
            "pool_gib": n_sets * per_set / (1 << 30), "gate_us": g_ms * 1e3, "down_us": d_ms * 1e3}


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


def moe_section(ctx, ev, rng, calls, n_layers=8, n_tokens=61):
    """MoE layer µs/token. Cold: calls rotate over n_layers layers (each with its
    own 64 experts, 158 MB) and, at batch 1, over n_tokens distinct tokens, so
    the routed experts change from call to call and the touched weights
    (about 0.6 GB at batch 1, 1 GB at batch 64) exceed the 256 MB
    Infinity Cache. Warm: one layer and one input repeated."""
    router, gate, up, down, shared = moe_weights(rng)
    h64, id_router = zipf_batch(rng, 64)
    kw = dict(hidden=HIDDEN, inter=INTER, n_experts=EXPERTS, expert_type=mm.IQ2_XXS, gate=gate, up=up, down=down,
              shared=shared, shared_inter=INTER)
    dec = [mm.MoeLayer(ctx, router=router, **kw) for _ in range(n_layers)]
    pre = [mm.MoeLayer(ctx, router=id_router, **kw) for _ in range(n_layers)]
    stream = ctx.stream
    toks = rng.standard_normal((n_tokens, HIDDEN)).astype(np.float32)
    cases = ((1, dec, [mm.DeviceArray.from_numpy(ctx, toks[j:j + 1]) for j in range(n_tokens)]),
             (64, pre, [mm.DeviceArray.from_numpy(ctx, h64)]))
    out, warm = {}, {}
    for t, layers, hs in cases:
        od = mm.DeviceArray(ctx, t * HIDDEN * 4)
        n = calls if t == 1 else max(10, calls // 4)
        n = max(n, 2 * n_layers)

        def run(i):
            layers[i % n_layers].ffn_dev(hs[i % len(hs)], od, t)

        for i in range(2 * n_layers):
            run(i)
        ctx.synchronize()
        out[t] = ev.time_ms(stream, lambda: [run(i) for i in range(n)]) / n * 1e3 / t
        for _ in range(5):
            layers[0].ffn_dev(hs[0], od, t)
        ctx.synchronize()
        warm[t] = ev.time_ms(stream, lambda: [layers[0].ffn_dev(hs[0], od, t) for _ in range(n)]) / n * 1e3 / t
        for h in hs:
            h.free()
        od.free()
    touched = len(set(np.argsort(-h64[:, :EXPERTS], axis=1)[:, :4].reshape(-1).tolist()))
    for layer in dec + pre:
        layer.free()
    return out, warm, touched, (router, gate, up, down, shared, h64, id_router)


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
        us = float(np.median([ev.time_ms(st, lambda: [fn() for _ in range(reps)]) / reps for _ in range(5)])) * 1e3
        gbs = (x.nbytes + nbytes) / (us * 1e-6) / 1e9
        out[name] = {"us": round(us, 2), "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}
    for a in (dx, db, dy):
        a.free()
    out["workload"] = (f"{n_rows} positions x {row_len} f32 (kv_lora 512 + rope 64) <-> Q8_0 blocks; "
                       f"{x.nbytes + nbytes} algorithmic bytes per kernel call")
    return out


def cpu_kv_codec_baseline(rng, seconds=2.0, row_len=576):
    """Oracle quantizeQ8_0 per row on one core (KVCache.put's loop), bounded sample."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc
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


def logits_section(ctx, ev, rng, reps=20, vocab=154880, hidden=HIDDEN):
    """computeLogits + sampleGreedy (inference.zig:1189-1197, 376-386): the
    output projection GEMV [vocab x hidden] in Q8_0 and IQ2_XXS (the GGUF's
    type decides), weights rotating over at least 300 MB, then the greedy
    argmax over the logits on the device."""
    x = mm.DeviceArray.from_numpy(ctx, rng.standard_normal(hidden).astype(np.float32))
    y = mm.DeviceArray(ctx, vocab * 4)
    tok = mm.DeviceArray(ctx, 4)
    st = ctx.stream
    out = {"workload": f"output projection [{vocab} x {hidden}] GEMV + greedy argmax over {vocab} logits"}
    for name, t in (("q8_0", mm.Q8_0), ("iq2_xxs", mm.IQ2_XXS)):
        raw = mm.make_weight(rng, t, vocab, hidden)
        n_sets = max(1, int(np.ceil(300e6 / raw.nbytes)))
        ws = [ctx.upload(raw, t, vocab, hidden) for _ in range(n_sets)]
        k = [0]

        def one():
            ctx.gemv_batched_dev(ws[k[0] % n_sets], 0, 1, x, 0, y, 0)
            k[0] += 1

        for _ in range(2 * n_sets):
            one()
        ctx.synchronize()
        us = float(np.median([ev.time_ms(st, lambda: [one() for _ in range(reps)]) / reps for _ in range(5)])) * 1e3
        nbytes = raw.nbytes + hidden * 4 + vocab * 4
        out[name] = {"us": round(us, 2), "GB/s": round(nbytes / (us * 1e-6) / 1e9, 1),
                     "frac": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4), "weight_bytes": int(raw.nbytes),
                     "copies": n_sets}
        for w in ws:
            w.free()
    for _ in range(3):
        ctx.argmax_dev(tok, y, vocab)
    ctx.synchronize()
    out["argmax_us"] = round(float(np.median([ev.time_ms(st, lambda: [ctx.argmax_dev(tok, y, vocab)
                                                                      for _ in range(reps)]) / reps
                                              for _ in range(5)])) * 1e3, 2)
    for a in (x, y, tok):
        a.free()
    return out


def mla_section(ctx, ev, rng, reps=20, n_layers=47, batch=64):
    """MLA attention projections (inference.zig:467-489, 663-665; batch path
    684-706, 880-882) on the same kernels: q_a [768 x 2048], q_b [3840 x 768],
    kv_a [576 x 2048], o_proj [2048 x 2560], one layer's four GEMVs per decode
    step with the weights of 47 layers rotating (cold, as in decode), and the
    four batched products at 64 tokens."""
    shapes = {"q_a": (768, 2048), "q_b": (3840, 768), "kv_a": (576, 2048), "o_proj": (2048, 2560)}
    st = ctx.stream
    xs = {n: mm.DeviceArray.from_numpy(ctx, rng.standard_normal(batch * c).astype(np.float32))
          for n, (_, c) in shapes.items()}
    ys = {n: mm.DeviceArray(ctx, batch * r * 4) for n, (r, _) in shapes.items()}
    ys["qkv_a"] = mm.DeviceArray(ctx, (768 + 576) * 4)
    out = {"workload": f"MLA projections of {n_layers} layers: " +
                       ", ".join(f"{n} [{r}x{c}]" for n, (r, c) in shapes.items()) +
                       f"; decode = the four GEMVs of one layer (fused: q_a and kv_a as one stacked weight), "
                       f"batch = the four products at {batch} tokens"}
    for name, t in (("q8_0", mm.Q8_0), ("iq2_xxs", mm.IQ2_XXS)):
        raws = {n: mm.make_weight(rng, t, r, c) for n, (r, c) in shapes.items()}
        layers = [{n: ctx.upload(raws[n], t, r, c) for n, (r, c) in shapes.items()} for _ in range(n_layers)]
        k = [0]

        def decode():
            lw = layers[k[0] % n_layers]
            for n in shapes:
                ctx.gemv_batched_dev(lw[n], 0, 1, xs[n], 0, ys[n], 0)
            k[0] += 1

        def prefill():
            lw = layers[k[0] % n_layers]
            for n in shapes:
                ctx.qmm_dev(lw[n], 0, xs[n], ys[n], batch)
            k[0] += 1

        # q_a and kv_a read the same hidden vector: one weight of 768 + 576
        # stacked rows (the raw rows concatenated), so three launches per layer.
        qkv = np.concatenate([raws["q_a"], raws["kv_a"]])
        fused = [ctx.upload(qkv, t, 768 + 576, 2048) for _ in range(n_layers)]

        def decode_fused():
            lw, i = layers[k[0] % n_layers], k[0] % n_layers
            ctx.gemv_batched_dev(fused[i], 0, 1, xs["q_a"], 0, ys["qkv_a"], 0)
            for n in ("q_b", "o_proj"):
                ctx.gemv_batched_dev(lw[n], 0, 1, xs[n], 0, ys[n], 0)
            k[0] += 1

        res = {}
        for label, fn in (("decode", decode), ("decode_fused_qkv_a", decode_fused), ("batch64", prefill)):
            for _ in range(n_layers):
                fn()
            ctx.synchronize()
            us = float(np.median([ev.time_ms(st, lambda: [fn() for _ in range(reps)]) / reps
                                  for _ in range(5)])) * 1e3
            res[label + "_us_per_layer"] = round(us, 2)
        wbytes = sum(int(r.nbytes) for r in raws.values())
        nbytes = wbytes + sum(4 * (r + c) for r, c in shapes.values())
        res["decode_GB/s"] = round(nbytes / (res["decode_us_per_layer"] * 1e-6) / 1e9, 1)
        res["decode_frac"] = round(res["decode_GB/s"] / HBM_PEAK_GBS, 4)
        res["weight_bytes_per_layer"] = wbytes
        out[name] = res
        for lw in layers:
            for w in lw.values():
                w.free()
        for w in fused:
            w.free()
    for a in list(xs.values()) + list(ys.values()):
        a.free()
    return out


def cpu_gemv_baseline(seconds):
    """Oracle IQ2_XXS GEMV (dequantize + f32 GEMV, one thread), bounded sample:
    alternating [1536 x 2048] and [2048 x 1536] matrices for about `seconds`."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc
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


def cpu_moe_baseline(weights, tokens):
    """Oracle moeFFN with the reference's 4-worker pool (5 threads with the
    caller), one call per token as forwardBatch does."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc
    router, gate, up, down, shared, h64, id_router = weights
    kw = dict(hidden=HIDDEN, inter=INTER, n_experts=EXPERTS, expert_type=orc.IQ2_XXS, gate=gate, up=up, down=down,
              shared=shared, shared_inter=INTER)
    pool = orc.Pool(4)
    try:
        moe = orc.Moe(router=router, **kw)
        h1 = np.random.default_rng(7).standard_normal((1, HIDDEN)).astype(np.float32)
        moe.ffn(h1, pool=pool)
        t0 = time.perf_counter()
        reps = 3
        for _ in range(reps):
            moe.ffn(h1, pool=pool)
        b1 = (time.perf_counter() - t0) / reps
        moe64 = orc.Moe(router=id_router, **kw)
        t0 = time.perf_counter()
        moe64.ffn(h64[:tokens], pool=pool)
        b64 = (time.perf_counter() - t0) / tokens
    finally:
        pool.close()
    return {"batch1_us_per_token": round(b1 * 1e6, 1), "batch64_us_per_token": round(b64 * 1e6, 1),
            "unit": "µs/token", "cores": 5, "kind": "port",
            "sample": f"{reps} batch-1 calls; the first {tokens} tokens of the batch-64 case, one moeFFN per token"}


def counter_pass():
    """Workload for the rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs: six
    launches of each IQ2_XXS GEMV shape, then three device-to-device copies of
    256 MiB (hipMemcpy's copy kernel) whose known size calibrates the counters."""
    ctx = mm.Context(0)
    rng = np.random.default_rng(1)
    gate = [ctx.upload(mm.make_iq2_xxs(rng, INTER, HIDDEN, EXPERTS), mm.IQ2_XXS, INTER, HIDDEN, EXPERTS)
            for _ in range(2)]
    down = [ctx.upload(mm.make_iq2_xxs(rng, HIDDEN, INTER, EXPERTS), mm.IQ2_XXS, HIDDEN, INTER, EXPERTS)
            for _ in range(2)]
    x = mm.DeviceArray.from_numpy(ctx, rng.standard_normal(HIDDEN).astype(np.float32))
    xd = mm.DeviceArray.from_numpy(ctx, rng.standard_normal((EXPERTS, INTER)).astype(np.float32))
    yg = mm.DeviceArray(ctx, EXPERTS * INTER * 4)
    yd = mm.DeviceArray(ctx, EXPERTS * HIDDEN * 4)
    for i in range(6):
        ctx.gemv_batched_dev(gate[i % 2], 0, EXPERTS, x, 0, yg, INTER)
    for i in range(6):
        ctx.gemv_batched_dev(down[i % 2], 0, EXPERTS, xd, INTER, yd, HIDDEN)
    ctx.synchronize()
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    nb = 256 << 20
    a, b = mm.DeviceArray(ctx, nb), mm.DeviceArray(ctx, nb)
    for _ in range(3):
        if hip.hipMemcpy(ctypes.c_void_p(b.ptr), ctypes.c_void_p(a.ptr), nb, 3) != 0:
            raise RuntimeError("hipMemcpy failed")
    ctx.close()
    print("counter pass done", flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--pool-gib", type=float, default=1.25)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--cpu-moe-tokens", type=int, default=8)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-moe", action="store_true")
    ap.add_argument("--counter-pass", action="store_true",
                    help="only run the workload of the FETCH_SIZE / WRITE_SIZE counter runs")
    args = ap.parse_args()
    if args.counter_pass:
        counter_pass()
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); "
              "this build has no multi-GPU path", file=sys.stderr)
        sys.exit(2)

    ctx = mm.Context(0)
    ev = HipEvents()
    rng = np.random.default_rng(1234)
    g = gemv_section(ctx, ev, mm.IQ2_XXS, args.steps, args.warmup, args.pool_gib, rng)
    value = g["step_bytes"] * args.steps / g["dt"] / 1e9
    kernel_us = g["gate_us"] + g["down_us"]
    achieved = g["step_bytes"] / (kernel_us * 1e-6) / 1e9
    traffic = read_traffic()
    q8 = gemv_section(ctx, ev, mm.Q8_0, max(20, args.steps // 4), max(5, args.warmup // 4), args.pool_gib, rng)

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
        "dtype": "int8",
        "data": "synthetic",
        "config": {
            "workload": "IQ2_XXS decode GEMV, batch 1: 64 expert matrices [1536x2048] (shared x) + "
                        "64 expert matrices [2048x1536] (one x each) per step, one launch per shape, "
                        f"weights rotating over {g['n_sets']} distinct copies ({g['pool_gib']:.2f} GiB)",
            "hidden": HIDDEN, "expert_inter": INTER, "experts_per_launch": EXPERTS,
            "bytes_per_step": g["step_bytes"],
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": (None if traffic is None else
                        round(traffic["gate_bytes_per_launch"] + traffic["down_bytes_per_launch"])),
            "kernel": "gemv_iq2_kernel, one launch per shape",
            "kernel_us_per_step": round(kernel_us, 3),
            "kernel_us": {"gate_1536x2048": round(g["gate_us"], 3), "down_2048x1536": round(g["down_us"], 3)},
            "bytes_per_step": g["step_bytes"],
        },
        "q8_gemv": {"value": round(q8["step_bytes"] * max(20, args.steps // 4) / q8["dt"] / 1e9, 2), "unit": "GB/s",
                    "kernel_us": {"gate_1536x2048": round(q8["gate_us"], 3), "down_2048x1536": round(q8["down_us"], 3)},
                    "achieved": round(q8["step_bytes"] / ((q8["gate_us"] + q8["down_us"]) * 1e-6) / 1e9, 1)},
    }
    weights = None
    if not args.no_moe:
        moe, warm, touched, weights = moe_section(ctx, ev, rng, max(50, args.steps))
        out["moe"] = {"batch1_us_per_token": round(moe[1], 3), "batch64_us_per_token": round(moe[64], 3),
                      "batch1_warm_us_per_token": round(warm[1], 3), "batch64_warm_us_per_token": round(warm[64], 3),
                      "unit": "µs/token", "experts_touched_batch64": touched,
                      "workload": "hidden 2048, 64 IQ2_XXS experts (1536) top-4 + shared, f32 router; "
                                  "batch 64 with Zipf(1.1) routing; cold: eight layers rotate (batch 1 also over "
                                  "61 tokens); warm: one layer, one input"}
    out["kv_q8_codec"] = kv_codec_section(ctx, ev, rng)
    out["logits"] = logits_section(ctx, ev, rng)
    out["mla"] = mla_section(ctx, ev, rng)
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_gemv_baseline(args.cpu_seconds)
        out["kv_q8_codec"]["cpu_quantize"] = cpu_kv_codec_baseline(rng)
        if weights is not None:
            out["cpu_moe"] = cpu_moe_baseline(weights, args.cpu_moe_tokens)
    ctx.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
