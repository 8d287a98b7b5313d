"""MoE FFN layer on the GPU against the oracle's moeFFN (inference.zig:886-1010).

Routing ids must equal the oracle's for every token: the router GEMV sums in
math.matVecMul's order (math.zig:79-99), so its scores are the CPU path's
bits and top-k sees the same values, near-ties and exact ties included.
Route weights: 1e-6 relative (expf on the GPU vs libm). Outputs: max-abs-rel
1e-3 (f32 accumulation of block-quantised products, as the GEMV tests).
"""
import numpy as np
import pytest

import mmhip as mm

pytestmark = pytest.mark.gpu

TOL_OUT = 1e-3
TOL_W = 1e-6


def _weights(rng, fmt, hidden, inter, n_exp, shared_inter=None, shared_fmt=None, router_sigma=0.02):
    router = rng.normal(0.0, router_sigma, (n_exp, hidden)).astype(np.float32)
    gate = mm.make_weight(rng, fmt, inter, hidden, n_exp)
    up = mm.make_weight(rng, fmt, inter, hidden, n_exp)
    down = mm.make_weight(rng, fmt, hidden, inter, n_exp)
    shared = None
    if shared_inter:
        sf = shared_fmt if shared_fmt is not None else fmt
        shared = (mm.make_weight(rng, sf, shared_inter, hidden), mm.make_weight(rng, sf, shared_inter, hidden),
                  mm.make_weight(rng, sf, hidden, shared_inter))
    return router, gate, up, down, shared


def _layers(ctx, orc, fmt, hidden, inter, n_exp, router, gate, up, down, shared, shared_inter=None,
            shared_fmt=None, rsf=1.0, bias=None):
    kw = dict(hidden=hidden, inter=inter, n_experts=n_exp, expert_type=fmt, router=router, gate=gate, up=up,
              down=down, shared=shared, shared_inter=shared_inter, shared_type=shared_fmt,
              routed_scaling_factor=rsf)
    gpu = mm.MoeLayer(ctx, **kw)
    cpu = orc.Moe(deferral_bias=bias, **kw)
    return gpu, cpu


def _check(orc, router, h, out_g, ids_g, w_g, out_c, ids_c, w_c):
    """Exact ids for every token, weights to TOL_W, outputs to TOL_OUT."""
    np.testing.assert_array_equal(ids_g, ids_c)
    np.testing.assert_allclose(w_g, w_c, rtol=TOL_W, atol=1e-7)
    err = mm.max_abs_rel(out_g, out_c)
    assert err < TOL_OUT, f"max-abs-rel {err:.3g}"
    return err


@pytest.mark.parametrize("fmt", ["iq2", "q8"])
def test_decode_glm_shape(ctx, orc, fmt):
    """One token through a GLM-4.7-Flash-shaped layer: hidden 2048, expert width
    1536, 64 routed experts top-4 plus a shared expert."""
    f = mm.IQ2_XXS if fmt == "iq2" else mm.Q8_0
    rng = np.random.default_rng(300 if fmt == "iq2" else 301)
    H, I, E = 2048, 1536, 64
    router, gate, up, down, shared = _weights(rng, f, H, I, E, shared_inter=I)
    gpu, cpu = _layers(ctx, orc, f, H, I, E, router, gate, up, down, shared, shared_inter=I)
    try:
        h = rng.standard_normal((1, H)).astype(np.float32)
        out_g, ids_g, w_g = gpu.ffn(h)
        out_c, ids_c, w_c = cpu.ffn(h)
        assert ids_g.shape == (1, 4)
        _check(orc, router, h, out_g, ids_g, w_g, out_c, ids_c, w_c)
    finally:
        gpu.free()


def _zipf_hidden(rng, t, hidden, n_exp, s=1.1):
    """Hidden states whose first n_exp coordinates are the router logits under
    an identity router: N(0, 1) with +10 on 4 distinct experts per token drawn
    from Zipf(s) over a seeded permutation of the experts."""
    perm = rng.permutation(n_exp)
    p = 1.0 / np.arange(1, n_exp + 1) ** s
    p /= p.sum()
    h = rng.standard_normal((t, hidden)).astype(np.float32)
    for ti in range(t):
        chosen = perm[rng.choice(n_exp, 4, replace=False, p=p)]
        h[ti, chosen] += 10.0
    router = np.zeros((n_exp, hidden), dtype=np.float32)
    router[:, :n_exp] = np.eye(n_exp, dtype=np.float32)
    return h, router


def test_prefill_zipf_batch64(ctx, orc):
    """64 tokens, skewed routing over 64 IQ2_XXS experts, grouped by expert."""
    rng = np.random.default_rng(310)
    H, I, E, T = 2048, 1536, 64, 64
    h, router = _zipf_hidden(rng, T, H, E)
    _, gate, up, down, shared = _weights(rng, mm.IQ2_XXS, H, I, E, shared_inter=I)
    gpu, cpu = _layers(ctx, orc, mm.IQ2_XXS, H, I, E, router, gate, up, down, shared, shared_inter=I)
    pool = orc.Pool(4)
    try:
        out_g, ids_g, w_g = gpu.ffn(h)
        out_c, ids_c, w_c = cpu.ffn(h, pool=pool)
        _check(orc, router, h, out_g, ids_g, w_g, out_c, ids_c, w_c)
        counts = np.bincount(ids_c.reshape(-1).astype(np.int64), minlength=E)
        assert counts.max() > 8  # the routing is skewed: one group spans several QMM rows
    finally:
        pool.close()
        gpu.free()


SMALL = dict(H=512, I=256, E=16)


def _small_case(ctx, orc, seed, fmt=mm.IQ2_XXS, shared_inter=256, shared_fmt=None, rsf=1.0, bias=None):
    rng = np.random.default_rng(seed)
    H, I, E = SMALL["H"], SMALL["I"], SMALL["E"]
    router, gate, up, down, shared = _weights(rng, fmt, H, I, E, shared_inter=shared_inter, shared_fmt=shared_fmt,
                                              router_sigma=0.05)
    gpu, cpu = _layers(ctx, orc, fmt, H, I, E, router, gate, up, down, shared, shared_inter=shared_inter,
                       shared_fmt=shared_fmt, rsf=rsf, bias=bias)
    return rng, router, gpu, cpu


@pytest.mark.parametrize("t", [1, 2, 3, 33, 64, 256])
def test_token_counts(ctx, orc, t):
    """Decode (1) and grouped prefill (2..256 = MMHIP_MOE_MAX_TOKENS) paths."""
    rng, router, gpu, cpu = _small_case(ctx, orc, 320 + t)
    try:
        h = rng.standard_normal((t, SMALL["H"])).astype(np.float32)
        out_g, ids_g, w_g = gpu.ffn(h)
        out_c, ids_c, w_c = cpu.ffn(h)
        _check(orc, router, h, out_g, ids_g, w_g, out_c, ids_c, w_c)
    finally:
        gpu.free()


@pytest.mark.parametrize("shared_inter", [256, 512])
def test_decode_calls_in_a_row(ctx, orc, shared_inter):
    """Decode calls back to back on one layer, a prefill call and a heavy-throttle
    call (one routed expert) in between: the routing outputs and problem lists
    the decode kernels leave in the layer's scratch are rewritten on every
    call, so every call must match the oracle. 512: the shared expert runs as
    separate launches."""
    rng, router, gpu, cpu = _small_case(ctx, orc, 390 + shared_inter, shared_inter=shared_inter)
    try:
        for t, level in ((1, 0), (1, 0), (3, 0), (1, 3), (1, 0), (1, 1)):
            h = rng.standard_normal((t, SMALL["H"])).astype(np.float32)
            out_g, ids_g, w_g = gpu.ffn(h, level=level)
            out_c, ids_c, w_c = cpu.ffn(h, level=level)
            _check(orc, router, h, out_g, ids_g, w_g, out_c, ids_c, w_c)
    finally:
        gpu.free()


@pytest.mark.parametrize("level", [0, 1, 2, 3])
@pytest.mark.parametrize("t", [1, 9])
def test_throttle_levels(ctx, orc, level, t):
    """ThrottleState levels: k = 4, 3, 2, 1 and routed scale 1, .83, .67, .5."""
    rng, router, gpu, cpu = _small_case(ctx, orc, 330 + level + 10 * t, rsf=1.5)
    try:
        h = rng.standard_normal((t, SMALL["H"])).astype(np.float32)
        out_g, ids_g, w_g = gpu.ffn(h, level=level)
        out_c, ids_c, w_c = cpu.ffn(h, level=level)
        assert ids_g.shape[1] == [4, 3, 2, 1][level]
        _check(orc, router, h, out_g, ids_g, w_g, out_c, ids_c, w_c)
    finally:
        gpu.free()


@pytest.mark.parametrize("t", [1, 5])
def test_heavy_fallback_with_deferral_bias(ctx, orc, t):
    """Heavy throttle with the expert limit raised to 4: only the top expert
    runs, renormalised to the routed scale, and the deferral bias is added."""
    bias = np.random.default_rng(77).normal(0, 0.1, SMALL["H"]).astype(np.float32)
    rng, router, gpu, cpu = _small_case(ctx, orc, 340 + t, bias=bias)
    try:
        h = rng.standard_normal((t, SMALL["H"])).astype(np.float32)
        out_g, ids_g, w_g = gpu.ffn(h, level=3, active_expert_limit=4, deferral_bias=bias)
        out_c, ids_c, w_c = cpu.ffn(h, level=3, active_expert_limit=4)
        assert ids_g.shape[1] == 4
        _check(orc, router, h, out_g, ids_g, w_g, out_c, ids_c, w_c)
        np.testing.assert_allclose(w_g[:, 0], 0.5, rtol=1e-6)
        # Without the bias the outputs differ by exactly that bias (within rounding).
        out_nb, _, _ = gpu.ffn(h, level=3, active_expert_limit=4)
        assert mm.max_abs_rel(out_g - out_nb, np.broadcast_to(bias, out_g.shape)) < 1e-4
    finally:
        gpu.free()


@pytest.mark.parametrize("t", [1, 7])
def test_q8_experts(ctx, orc, t):
    rng, router, gpu, cpu = _small_case(ctx, orc, 350 + t, fmt=mm.Q8_0)
    try:
        h = rng.standard_normal((t, SMALL["H"])).astype(np.float32)
        out_g, ids_g, w_g = gpu.ffn(h)
        out_c, ids_c, w_c = cpu.ffn(h)
        _check(orc, router, h, out_g, ids_g, w_g, out_c, ids_c, w_c)
    finally:
        gpu.free()


@pytest.mark.parametrize("t", [1, 6])
@pytest.mark.parametrize("variant", ["wider", "other_type", "none"])
def test_shared_expert_variants(ctx, orc, t, variant):
    """Shared expert of another width or type (separate launches) or absent."""
    shared_inter = {"wider": 512, "other_type": 256, "none": None}[variant]
    shared_fmt = mm.Q8_0 if variant == "other_type" else None
    rng, router, gpu, cpu = _small_case(ctx, orc, 360 + t, shared_inter=shared_inter, shared_fmt=shared_fmt)
    try:
        h = rng.standard_normal((t, SMALL["H"])).astype(np.float32)
        out_g, ids_g, w_g = gpu.ffn(h)
        out_c, ids_c, w_c = cpu.ffn(h)
        _check(orc, router, h, out_g, ids_g, w_g, out_c, ids_c, w_c)
    finally:
        gpu.free()


def test_expert_counts_follow_stats(ctx, orc):
    """ExpertStats.counts: every selected expert of every call (skipped ones
    included), accumulated over calls."""
    rng, router, gpu, cpu = _small_case(ctx, orc, 370)
    stats = orc.Stats(1, SMALL["E"])
    try:
        for t, level in ((1, 0), (11, 0), (4, 2), (3, 3)):
            h = rng.standard_normal((t, SMALL["H"])).astype(np.float32)
            gpu.ffn(h, level=level)
            cpu.ffn(h, level=level, stats=stats)
        np.testing.assert_array_equal(gpu.expert_counts(), stats.counts[:SMALL["E"]])
    finally:
        gpu.free()


def test_device_twin_matches_host_call(ctx, orc):
    rng, router, gpu, cpu = _small_case(ctx, orc, 380)
    try:
        t = 12
        h = rng.standard_normal((t, SMALL["H"])).astype(np.float32)
        out_h, _, _ = gpu.ffn(h)
        hd = mm.DeviceArray.from_numpy(ctx, h)
        od = mm.DeviceArray(ctx, h.nbytes)
        gpu.ffn_dev(hd, od, t)
        ctx.synchronize()
        assert np.array_equal(od.to_numpy(np.float32, h.size).reshape(h.shape), out_h)
    finally:
        gpu.free()


def test_invalid_calls(ctx, orc):
    rng, router, gpu, cpu = _small_case(ctx, orc, 390)
    try:
        with pytest.raises(mm.MmhipError):
            gpu.ffn(np.zeros((0, SMALL["H"]), np.float32))
        with pytest.raises(mm.MmhipError):
            gpu.ffn(np.zeros((257, SMALL["H"]), np.float32))
        # ThrottleLevel has four values (thermal.zig:10-15): others are errors,
        # not an unthrottled call.
        h = rng.standard_normal((1, SMALL["H"])).astype(np.float32)
        for bad in (-1, 4, 7):
            with pytest.raises(mm.MmhipError, match="throttle_level"):
                gpu.ffn(h, level=bad)
    finally:
        gpu.free()


@pytest.mark.parametrize("n_exp", [128, 256])
@pytest.mark.parametrize("t", [1, 24])
def test_many_experts(ctx, orc, n_exp, t):
    """More than 64 experts (up to the 256 the routing kernels hold), decode and
    grouped prefill, with distinct router logits and then with identity-router
    scores from four values (ties at the k-th place, heap order)."""
    rng = np.random.default_rng(450 + n_exp + t)
    H, I = 256, 256
    router, gate, up, down, shared = _weights(rng, mm.IQ2_XXS, H, I, n_exp, shared_inter=I, router_sigma=0.05)
    gpu, cpu = _layers(ctx, orc, mm.IQ2_XXS, H, I, n_exp, router, gate, up, down, shared, shared_inter=I)
    try:
        h = rng.standard_normal((t, H)).astype(np.float32)
        out_g, ids_g, w_g = gpu.ffn(h)
        out_c, ids_c, w_c = cpu.ffn(h)
        _check(orc, router, h, out_g, ids_g, w_g, out_c, ids_c, w_c)
    finally:
        gpu.free()
    ident = np.zeros((n_exp, H), dtype=np.float32)
    ident[:, :n_exp] = np.eye(n_exp, dtype=np.float32)
    gpu, cpu = _layers(ctx, orc, mm.IQ2_XXS, H, I, n_exp, ident, gate, up, down, shared, shared_inter=I)
    try:
        h = rng.standard_normal((t, H)).astype(np.float32)
        h[:, :n_exp] = rng.choice(np.array([-1.0, 0.0, 0.5, 1.0], dtype=np.float32), (t, n_exp))
        out_g, ids_g, w_g = gpu.ffn(h)
        out_c, ids_c, w_c = cpu.ffn(h)
        np.testing.assert_array_equal(ids_g, ids_c)
        np.testing.assert_allclose(w_g, w_c, rtol=TOL_W, atol=1e-7)
        assert mm.max_abs_rel(out_g, out_c) < TOL_OUT
    finally:
        gpu.free()


@pytest.mark.parametrize("level", [0, 2, 3])
def test_decode_routing_ties_follow_the_heap(ctx, orc, level):
    """Decode calls (one token each, routed inside the gate/up kernel) under an
    identity router: four-valued scores that tie at the k-th place, a token
    whose two largest scores are +0 and -0 (equal as floats, so the heap's
    insertion order decides), a NaN score past the heap's seed positions, and
    distinct scores. Ids and their order must be math.topK's
    (math.zig:130-174)."""
    rng = np.random.default_rng(420 + level)
    H, I, E = 512, 256, 64
    _, gate, up, down, shared = _weights(rng, mm.IQ2_XXS, H, I, E, shared_inter=I)
    router = np.zeros((E, H), dtype=np.float32)
    router[:, :E] = np.eye(E, dtype=np.float32)
    rows = [rng.choice(np.array([-1.0, 0.0, 0.5, 1.0], dtype=np.float32), E) for _ in range(10)]
    zeros = (-1.0 - rng.random(E)).astype(np.float32)
    zeros[[9, 3]] = np.array([-0.0, 0.0], dtype=np.float32)
    rows += [zeros, zeros[::-1].copy(), rng.standard_normal(E).astype(np.float32)]
    # Expert 37's router row also reads a column past the identity block with
    # a NaN weight: only its score is NaN.
    nan_router = router.copy()
    nan_router[37, E + 5] = np.nan
    for rt, rr in ((router, rows), (nan_router, rows[:2] + rows[-1:])):
        gpu, cpu = _layers(ctx, orc, mm.IQ2_XXS, H, I, E, rt, gate, up, down, shared, shared_inter=I)
        try:
            for r in rr:
                h = rng.standard_normal((1, H)).astype(np.float32)
                h[0, :E] = r
                out_g, ids_g, w_g = gpu.ffn(h, level=level)
                out_c, ids_c, w_c = cpu.ffn(h, level=level)
                np.testing.assert_array_equal(ids_g, ids_c)
                np.testing.assert_allclose(w_g, w_c, rtol=TOL_W, atol=1e-7)
                assert mm.max_abs_rel(out_g, out_c) < TOL_OUT
        finally:
            gpu.free()


@pytest.mark.parametrize("level", [0, 1, 2, 3])
def test_routing_ties_follow_the_heap(ctx, orc, level):
    """Exact score ties: under an identity router the scores are the hidden
    states' first E coordinates, bit-identical on both sides, drawn from four
    values so that most tokens tie at the k-th place. The selected ids and
    their order must be the min-heap's (math.zig:130-174), not a sort's."""
    rng = np.random.default_rng(400 + level)
    H, I, E, T = 512, 256, 64, 64
    _, gate, up, down, shared = _weights(rng, mm.IQ2_XXS, H, I, E, shared_inter=I)
    router = np.zeros((E, H), dtype=np.float32)
    router[:, :E] = np.eye(E, dtype=np.float32)
    h = rng.standard_normal((T, H)).astype(np.float32)
    h[:, :E] = rng.choice(np.array([-1.0, 0.0, 0.5, 1.0], dtype=np.float32), (T, E))
    gpu, cpu = _layers(ctx, orc, mm.IQ2_XXS, H, I, E, router, gate, up, down, shared, shared_inter=I)
    try:
        out_g, ids_g, w_g = gpu.ffn(h, level=level)
        out_c, ids_c, w_c = cpu.ffn(h, level=level)
        np.testing.assert_array_equal(ids_g, ids_c)
        np.testing.assert_allclose(w_g, w_c, rtol=TOL_W, atol=1e-7)
        assert mm.max_abs_rel(out_g, out_c) < TOL_OUT
        # the ties are real: the k-th and (k+1)-th scores are equal for most tokens
        k = ids_c.shape[1]
        srt = -np.sort(-h[:, :E], axis=1)
        assert (srt[:, k - 1] == srt[:, k]).mean() > 0.5
    finally:
        gpu.free()


def _one_ulp_router(orc, rng, H, E, k=4):
    """A router and a hidden vector whose k-th and (k+1)-th scores differ by
    one ulp under math.matVecMul's order, while their exact (float64) dot
    products rank the two experts the other way round, so any other
    summation order (a tree, fused multiply-adds) is likely to pick the other
    expert. Row b (the (k+1)-th) is rescaled by factors 1 + 5e-9 j until its
    rounded score lands next to row a's."""
    for _ in range(20):
        router = rng.normal(0.0, 0.02, (E, H)).astype(np.float32)
        h = rng.standard_normal(H).astype(np.float32)
        sc = orc.matvec_f32(router, h, E, H)
        order = np.argsort(-sc, kind="stable")
        a, b = int(order[k - 1]), int(order[k])
        s_a = sc[a]
        base = router[b].astype(np.float64) * (float(s_a) / float(sc[b]))
        for j in range(-2000, 2001):
            row = (base * (1.0 + 5e-9 * j)).astype(np.float32)
            s_b = orc.matvec_f32(row[None, :], h, 1, H)[0]
            if abs(int(s_b.view(np.int32)) - int(s_a.view(np.int32))) != 1:
                continue
            exact_b = float(row.astype(np.float64) @ h.astype(np.float64))
            exact_a = float(router[a].astype(np.float64) @ h.astype(np.float64))
            others = np.delete(sc, [a, b])
            if (exact_b > exact_a) == (s_b > s_a) or np.any((others >= min(s_a, s_b)) & (others <= max(s_a, s_b))):
                continue
            r2 = router.copy()
            r2[b] = row
            return r2, h, a, b
    raise AssertionError("no one-ulp case found")


@pytest.mark.parametrize("t", [1, 20])
def test_one_ulp_near_tie_routes_exactly(ctx, orc, t):
    """The k-th and (k+1)-th router scores one ulp apart, in the opposite order
    from their exact values: the device must still pick the CPU path's
    experts, in decode (t = 1, routed in the gate/up kernel) and in a
    prefill batch (the crafted token at several positions among random
    ones, routed by the batch route kernel)."""
    rng = np.random.default_rng(777 + t)
    H, I, E = 2048, 256, 64
    router, hv, a, b = _one_ulp_router(orc, rng, H, E)
    _, gate, up, down, shared = _weights(rng, mm.IQ2_XXS, H, I, E, shared_inter=I)
    gpu, cpu = _layers(ctx, orc, mm.IQ2_XXS, H, I, E, router, gate, up, down, shared, shared_inter=I)
    try:
        h = rng.standard_normal((t, H)).astype(np.float32)
        for pos in {0, t // 3, t - 1}:
            h[pos] = hv
        out_g, ids_g, w_g = gpu.ffn(h)
        out_c, ids_c, w_c = cpu.ffn(h)
        sc = orc.matvec_f32(router, hv, E, H)
        assert abs(int(sc[a].view(np.int32)) - int(sc[b].view(np.int32))) == 1
        winner = a if sc[a] > sc[b] else b
        assert winner in ids_c[0] and (a if winner == b else b) not in ids_c[0]
        _check(orc, router, h, out_g, ids_g, w_g, out_c, ids_c, w_c)
    finally:
        gpu.free()
