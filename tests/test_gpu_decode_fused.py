"""One-launch decode MoE layer (decode_moe.hip) against the three-launch
sequence and the oracle's moeFFN (inference.zig:886-1010).

The one-launch kernel uses the same arithmetic in the same order as the
router GEMV, the routing gate/up GEMV and the down + combine launch, so its
output must equal theirs bit for bit: a layer built with
MMHIP_DECODE_FUSED=0 runs the three launches on the same weights. Calls run
back to back with different tokens and throttle levels, alternating between
the two layers, so counters left behind by one call would show in the next.
Against the oracle: route ids exact, weights 1e-6, outputs max-abs-rel 1e-3
(as tests/test_gpu_moe.py).
"""
import os
import types

import numpy as np
import pytest

import mmhip as mm

pytestmark = pytest.mark.gpu

TOL_OUT = 1e-3
TOL_W = 1e-6


def _weights(rng, hidden, inter, n_exp, shared, router_type=mm.F32):
    router = rng.normal(0.0, 0.02, (n_exp, hidden)).astype(np.float32)
    if router_type == mm.F16:
        router = router.astype(np.float16)
    gate = mm.make_weight(rng, mm.IQ2_XXS, inter, hidden, n_exp)
    up = mm.make_weight(rng, mm.IQ2_XXS, inter, hidden, n_exp)
    down = mm.make_weight(rng, mm.IQ2_XXS, hidden, inter, n_exp)
    sh = None
    if shared:
        sh = (mm.make_weight(rng, mm.IQ2_XXS, inter, hidden), mm.make_weight(rng, mm.IQ2_XXS, inter, hidden),
              mm.make_weight(rng, mm.IQ2_XXS, hidden, inter))
    return router, gate, up, down, sh


def _pair(ctx, hidden, inter, n_exp, router, gate, up, down, shared, router_type=mm.F32):
    """(one-launch layer, three-launch layer) on the same weights."""
    kw = dict(hidden=hidden, inter=inter, n_experts=n_exp, expert_type=mm.IQ2_XXS, router=router, gate=gate, up=up,
              down=down, shared=shared, shared_inter=inter if shared is not None else None,
              shared_type=mm.IQ2_XXS if shared is not None else None, routed_scaling_factor=1.8,
              router_type=router_type)
    prev = os.environ.pop("MMHIP_DECODE_FUSED", None)
    try:
        fused = mm.MoeLayer(ctx, **kw)
        os.environ["MMHIP_DECODE_FUSED"] = "0"
        split = mm.MoeLayer(ctx, **kw)
    finally:
        os.environ.pop("MMHIP_DECODE_FUSED", None)
        if prev is not None:
            os.environ["MMHIP_DECODE_FUSED"] = prev
    return fused, split, kw


def _same_bits(a, b):
    np.testing.assert_array_equal(np.ascontiguousarray(a).view(np.uint32), np.ascontiguousarray(b).view(np.uint32))


def _run_pair(ctx, orc, fused, split, kw, rng, calls, hidden, bias):
    cpu = orc.Moe(deferral_bias=bias, **kw)
    ctx.profile(True)
    for i, (level, limit) in enumerate(calls):
        h = rng.standard_normal((1, hidden)).astype(np.float32)
        db = bias if level == 3 else None
        out_f, ids_f, w_f = fused.ffn(h, level=level, active_expert_limit=limit, deferral_bias=db)
        out_s, ids_s, w_s = split.ffn(h, level=level, active_expert_limit=limit, deferral_bias=db)
        _same_bits(out_f, out_s)
        np.testing.assert_array_equal(ids_f, ids_s)
        _same_bits(w_f, w_s)
        if i < 2 or level == 3:
            out_c, ids_c, w_c = cpu.ffn(h, level=level, active_expert_limit=limit)
            np.testing.assert_array_equal(ids_f, ids_c)
            np.testing.assert_allclose(w_f, w_c, rtol=TOL_W, atol=1e-7)
            err = mm.max_abs_rel(out_f, out_c)
            assert err < TOL_OUT, f"call {i} level {level}: max-abs-rel {err:.3g}"
    _, n_fused = ctx.profile_read("moe_decode")
    _, n_router = ctx.profile_read("moe_router")
    ctx.profile(False)
    # Every fused call was one moe_decode launch; the split layer's calls
    # launched the router separately.
    assert n_fused == len(calls)
    assert n_router == len(calls)
    np.testing.assert_array_equal(fused.expert_counts(), split.expert_counts())


@pytest.mark.parametrize("shared", [True, False])
def test_one_launch_decode_glm_shape_matches_three_launches(ctx, orc, shared):
    """GLM-4.7-Flash shape: hidden 2048, expert width 1536, 64 experts, top-4
    (top-3/2/1 under throttle), merged shared expert or none."""
    rng = np.random.default_rng(700 + shared)
    H, I, E = 2048, 1536, 64
    router, gate, up, down, sh = _weights(rng, H, I, E, shared)
    fused, split, kw = _pair(ctx, H, I, E, router, gate, up, down, sh)
    bias = rng.normal(0.0, 0.5, H).astype(np.float32)
    try:
        # (throttle level, active expert limit): top-4/3/2/1, the heavy
        # fallback with deferral bias (level 3, limit 4), a limit of 2.
        calls = [(0, 0), (0, 0), (1, 0), (2, 0), (3, 4), (0, 0), (3, 0), (0, 2)]
        _run_pair(ctx, orc, fused, split, kw, rng, calls, H, bias)
    finally:
        fused.free()
        split.free()


def test_one_launch_decode_small_shape_f16_router(ctx, orc):
    """hidden 512, width 256, 16 experts, f16 router weights."""
    rng = np.random.default_rng(710)
    H, I, E = 512, 256, 16
    router, gate, up, down, sh = _weights(rng, H, I, E, True, router_type=mm.F16)
    fused, split, kw = _pair(ctx, H, I, E, router, gate, up, down, sh, router_type=mm.F16)
    bias = rng.normal(0.0, 0.5, H).astype(np.float32)
    try:
        _run_pair(ctx, orc, fused, split, kw, rng, [(0, 0), (1, 0), (0, 0), (3, 4), (2, 0), (0, 0)], H, bias)
    finally:
        fused.free()
        split.free()


def test_one_launch_decode_many_calls_in_a_row(ctx):
    """100 calls back to back on the device path (no host sync in between),
    then every output against the three-launch layer's."""
    rng = np.random.default_rng(720)
    H, I, E = 2048, 1536, 64
    router, gate, up, down, sh = _weights(rng, H, I, E, True)
    fused, split, _ = _pair(ctx, H, I, E, router, gate, up, down, sh)
    n = 100
    hs = rng.standard_normal((n, H)).astype(np.float32)
    x = mm.DeviceArray.from_numpy(ctx, hs)
    of = mm.DeviceArray(ctx, n * H * 4)
    os_ = mm.DeviceArray(ctx, n * H * 4)
    at = lambda d, i: types.SimpleNamespace(ptr=d.ptr + i * H * 4)  # row i of a device array
    try:
        for i in range(n):
            fused.ffn_dev(at(x, i), at(of, i), 1)
        for i in range(n):
            split.ffn_dev(at(x, i), at(os_, i), 1)
        ctx.synchronize()
        _same_bits(of.to_numpy(np.float32, n * H), os_.to_numpy(np.float32, n * H))
    finally:
        x.free()
        of.free()
        os_.free()
        fused.free()
        split.free()


@pytest.mark.parametrize("n_exp,shared,router_type", [(128, True, mm.F32), (256, False, mm.F16)])
def test_one_launch_decode_many_experts(ctx, orc, n_exp, shared, router_type):
    """128 and 256 routed experts (top-k over 2 or 4 score slots per lane),
    hidden 1024, width 512."""
    rng = np.random.default_rng(730 + n_exp)
    H, I = 1024, 512
    router, gate, up, down, sh = _weights(rng, H, I, n_exp, shared, router_type=router_type)
    fused, split, kw = _pair(ctx, H, I, n_exp, router, gate, up, down, sh, router_type=router_type)
    bias = rng.normal(0.0, 0.5, H).astype(np.float32)
    try:
        _run_pair(ctx, orc, fused, split, kw, rng, [(0, 0), (0, 0), (2, 0), (3, 4)], H, bias)
    finally:
        fused.free()
        split.free()


def test_one_launch_decode_wait_timeout_is_reported(ctx):
    """A grid-wide wait that gives up is reported, not silent: with
    MMHIP_DECODE_WAIT_US=0 each wait polls once, so workgroups that reach
    the routing before the router rows are published give up (the launch
    still ends). The call returns the HIP error code with the reason, the
    context's status is cleared, and a layer with the default limit then
    matches the three-launch path."""
    rng = np.random.default_rng(740)
    H, I, E = 2048, 1536, 64
    router, gate, up, down, sh = _weights(rng, H, I, E, True)
    kw = dict(hidden=H, inter=I, n_experts=E, expert_type=mm.IQ2_XXS, router=router, gate=gate, up=up, down=down,
              shared=sh, shared_inter=I, shared_type=mm.IQ2_XXS)
    prev = os.environ.pop("MMHIP_DECODE_WAIT_US", None)
    os.environ["MMHIP_DECODE_WAIT_US"] = "0"
    try:
        hasty = mm.MoeLayer(ctx, **kw)
    finally:
        os.environ.pop("MMHIP_DECODE_WAIT_US", None)
        if prev is not None:
            os.environ["MMHIP_DECODE_WAIT_US"] = prev
    fused, split, _ = _pair(ctx, H, I, E, router, gate, up, down, sh)
    try:
        errors = []
        for _ in range(10):
            h = rng.standard_normal((1, H)).astype(np.float32)
            try:
                hasty.ffn(h)
            except mm.MmhipError as e:
                errors.append(e)
        assert errors, "no wait gave up with a limit of one poll"
        assert all(e.code == -4 and "grid-wide wait" in str(e) for e in errors), errors[0]
        ctx.synchronize()  # the status word was cleared by the call that reported it
        h = rng.standard_normal((1, H)).astype(np.float32)
        _same_bits(fused.ffn(h)[0], split.ffn(h)[0])
    finally:
        hasty.free()
        fused.free()
        split.free()
