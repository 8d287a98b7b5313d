"""Benchmark: IQ2_XXS decode GEMV HBM bandwidth on one MI355X.

Workload (one step): the batch-1 decode GEMV of a GLM-4.7-Flash-shaped MoE
layer's routed experts, IQ2_XXS weights:
  launch 1: 64 expert gate projections W[1536 x 2048], one shared input x[2048]
  launch 2: 64 expert down projections W[2048 x 1536], one input per expert
Weights rotate over a pool of distinct device copies (> 1 GiB, several times
the 256 MiB Infinity Cache), so every step streams its weights from HBM.

Reported:
  value        whole-step algorithmic bytes / step time (GB/s), synchronize-
               bracketed wall time over --steps steps;
  roofline     the GEMV kernel alone: algorithmic bytes per launch / mean
               kernel duration from HIP events on the library stream, against
               the 8 TB/s HBM peak;
  cpu_baseline the oracle's CPU path (reference algorithm: dequantize the
               matrix to f32, then the 4-lane f32 GEMV) on one host core.
"""
import argparse
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


def gemv_bytes(rows, cols, n_mats, shared_x):
    w = mm.tensor_bytes(mm.IQ2_XXS, rows, cols) * n_mats
    x = cols * 4 * (1 if shared_x else n_mats)
    y = rows * 4 * n_mats
    return w + x + y


def cpu_baseline(seconds=10.0):
    """Oracle IQ2_XXS GEMV (dequantize + f32 GEMV, one thread) on a bounded
    sample: alternating [1536 x 2048] and [2048 x 1536] matrices for about
    `seconds` of CPU time."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc
    rng = np.random.default_rng(99)
    mats = [(mm.make_iq2_xxs(rng, INTER, HIDDEN), INTER, HIDDEN), (mm.make_iq2_xxs(rng, HIDDEN, INTER), HIDDEN, INTER)]
    xs = [rng.standard_normal(HIDDEN).astype(np.float32), rng.standard_normal(INTER).astype(np.float32)]
    n = 0
    nbytes = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        raw, r, c = mats[n % 2]
        orc.mat_vec_mul_unified(raw, orc.IQ2_XXS, xs[n % 2], r, c)
        nbytes += gemv_bytes(r, c, 1, True)
        n += 1
    dt = time.perf_counter() - t0
    return {"value": round(nbytes / dt / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{n} IQ2_XXS GEMVs alternating [1536x2048]/[2048x1536] in {dt:.1f} s, "
                      f"{dt / n * 1e6:.0f} us per GEMV"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--pool-gib", type=float, default=1.25)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); "
              "this build has no multi-GPU path", file=sys.stderr)
        sys.exit(2)

    ctx = mm.Context(0)
    rng = np.random.default_rng(1234)
    raw_gate = mm.make_iq2_xxs(rng, INTER, HIDDEN, EXPERTS)
    raw_down = mm.make_iq2_xxs(rng, HIDDEN, INTER, EXPERTS)
    per_set = 2 * mm.tensor_bytes(mm.IQ2_XXS, INTER, HIDDEN, EXPERTS)
    n_sets = max(2, int(args.pool_gib * (1 << 30) // per_set))
    sets = []
    for _ in range(n_sets):
        sets.append((ctx.upload(raw_gate, mm.IQ2_XXS, INTER, HIDDEN, EXPERTS),
                     ctx.upload(raw_down, mm.IQ2_XXS, HIDDEN, INTER, EXPERTS)))
    del raw_gate, raw_down
    x = mm.DeviceArray.from_numpy(ctx, rng.standard_normal(HIDDEN).astype(np.float32))
    xd = mm.DeviceArray.from_numpy(ctx, rng.standard_normal((EXPERTS, INTER)).astype(np.float32))
    yg = mm.DeviceArray(ctx, EXPERTS * INTER * 4)
    yd = mm.DeviceArray(ctx, EXPERTS * HIDDEN * 4)

    def step(i):
        g, d = sets[i % n_sets]
        ctx.gemv_batched_dev(g, 0, EXPERTS, x, 0, yg, INTER)
        ctx.gemv_batched_dev(d, 0, EXPERTS, xd, INTER, yd, HIDDEN)

    b_gate = gemv_bytes(INTER, HIDDEN, EXPERTS, True)
    b_down = gemv_bytes(HIDDEN, INTER, EXPERTS, False)
    step_bytes = b_gate + b_down

    for i in range(args.warmup):
        step(i)
    ctx.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(i)
    ctx.synchronize()
    dt = time.perf_counter() - t0
    ms_per_step = dt / args.steps * 1e3
    value = step_bytes / (dt / args.steps) / 1e9

    # Kernel-only timing of the GEMV launches (separate pass: events off above).
    ctx.profile(True)
    for i in range(args.steps):
        step(i)
    ms, launches = ctx.profile_read("gemv_q")
    ctx.profile(False)
    mean_launch_ms = ms / launches
    achieved = (step_bytes / 2) / (mean_launch_ms * 1e-3) / 1e9

    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {
            "workload": "IQ2_XXS decode GEMV, batch 1: 64 expert matrices [1536x2048] (shared x) + "
                        "64 expert matrices [2048x1536] (one x each) per step, one launch per shape, "
                        f"weights rotating over {n_sets} distinct copies "
                        f"({n_sets * per_set / (1 << 30):.2f} GiB)",
            "hidden": HIDDEN, "expert_inter": INTER, "experts_per_launch": EXPERTS,
            "bytes_per_step": step_bytes,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
            "kernel": "gemv_q_kernel<IQ2_XXS>",
            "mean_launch_us": round(mean_launch_ms * 1e3, 3),
            "bytes_per_launch": step_bytes // 2,
        },
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    for g, d in sets:
        g.free()
        d.free()
    ctx.close()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
