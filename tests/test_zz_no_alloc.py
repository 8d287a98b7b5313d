"""mmhip_qmm_dev_noalloc: the batched QMM (batchMatMulUnified's device twin)
with the library's fixed per-device scratch instead of an allocated one.

Its output must equal mmhip_qmm_dev's bit for bit (same kernels, same
inputs) on two calls in a row, the second with a smaller input, so that
nothing left in the shared scratch by the first call leaks into the second;
both are also checked against the oracle's matMulQ8_0 / dequantize + GEMV
(qmm.zig:58-138, inference.zig:1231-1264) at the QMM tolerance. Inputs beyond
the fixed scratch are refused with an error.
"""
import numpy as np
import pytest

import mmhip as mm

pytestmark = pytest.mark.gpu

TOL_QMM = 1e-2


def _run(ctx, fn, w, x, rows, batch, layout):
    dx = mm.DeviceArray.from_numpy(ctx, x)
    dy = mm.DeviceArray(ctx, rows * batch * 4)
    try:
        fn(w, 0, dx, dy, batch, layout)
        ctx.synchronize()
        y = dy.to_numpy(np.float32, rows * batch)
    finally:
        dx.free()
        dy.free()
    return y.reshape(batch, rows) if layout == 0 else y.reshape(rows, batch).T


@pytest.mark.parametrize("fmt", [mm.Q8_0, mm.IQ2_XXS])
@pytest.mark.parametrize("layout", [0, 1])
def test_noalloc_matches_qmm_dev_twice(ctx, orc, fmt, layout):
    rng = np.random.default_rng(900 + fmt + layout)
    cases = [(1536, 2048, 64), (512, 768, 5)]  # the second call is smaller in rows, columns and batch
    for rows, cols, batch in cases:
        raw = mm.make_weight(rng, fmt, rows, cols)
        x = (rng.standard_normal((batch, cols)) * 2.0).astype(np.float32)
        w = ctx.upload(raw, fmt, rows, cols)
        try:
            got = _run(ctx, ctx.qmm_dev_noalloc, w, x, rows, batch, layout)
            ref = _run(ctx, ctx.qmm_dev, w, x, rows, batch, layout)
        finally:
            w.free()
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (rows, cols, batch)
        cpu = orc.batch_mat_mul_unified(raw, fmt, x, rows, batch, cols).reshape(batch, rows)
        assert mm.max_abs_rel(got, cpu) <= TOL_QMM


def test_noalloc_size_limit(ctx):
    rng = np.random.default_rng(950)
    raw = mm.make_weight(rng, mm.IQ2_XXS, 16, 8448)  # 8448 columns: 256 x 8448 x 2.125 bytes > the scratch
    w = ctx.upload(raw, mm.IQ2_XXS, 16, 8448)
    dx = mm.DeviceArray.from_numpy(ctx, np.zeros((256, 8448), np.float32))
    dy = mm.DeviceArray(ctx, 256 * 16 * 4)
    try:
        with pytest.raises(mm.MmhipError, match="scratch"):
            ctx.qmm_dev_noalloc(w, 0, dx, dy, 256, 0)
        ctx.qmm_dev_noalloc(w, 0, dx, dy, 240, 0)  # 240 x 8448 x 2.125 fits
        ctx.synchronize()
    finally:
        w.free()
        dx.free()
        dy.free()


def test_noalloc_at_the_limit(ctx, orc):
    """256 vectors of 8192 columns fill the scratch exactly."""
    rng = np.random.default_rng(960)
    rows, cols, batch = 48, 8192, 256
    raw = mm.make_weight(rng, mm.Q8_0, rows, cols)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    w = ctx.upload(raw, mm.Q8_0, rows, cols)
    try:
        got = _run(ctx, ctx.qmm_dev_noalloc, w, x, rows, batch, 0)
        ref = _run(ctx, ctx.qmm_dev, w, x, rows, batch, 0)
    finally:
        w.free()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
