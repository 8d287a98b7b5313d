"""GPU parity of the decode GEMV and batched QMM against the oracle
(qmm.zig:13-138, math.zig:79-99, inference.zig:1200-1264). Tolerance:
max|y - ref| / max|ref| <= 1e-3 for the f32-accumulating GEMV paths and
1e-2 for the MFMA QMM path (the path's stated bars); the 16-bit block
fixed-point activations keep both far below that (~2e-5)."""
import threading

import numpy as np
import pytest

import mmhip as mm

pytestmark = pytest.mark.gpu

TOL_GEMV = 1e-3
TOL_QMM = 1e-2


def _weights(rng, t, rows, cols, count=1):
    return mm.make_weight(rng, t, rows, cols, count)


@pytest.mark.parametrize("t", [mm.Q8_0, mm.IQ2_XXS])
@pytest.mark.parametrize("rows,cols", [(1536, 2048), (2048, 1536)])
def test_gemv_config_shapes(ctx, orc, t, rows, cols):
    rng = np.random.default_rng(rows * 3 + t)
    raw = _weights(rng, t, rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    ref = orc.mat_vec_mul_unified(raw, t, x, rows, cols)
    got = ctx.mat_vec_mul(raw, t, x, rows, cols)
    err = mm.max_abs_rel(got, ref)
    print(f"type={t} {rows}x{cols} max_abs_rel={err:.3e}")
    assert err <= TOL_GEMV


def _bits_equal(got, ref):
    """Bit-exact comparison of float results (NaN-free data)."""
    got = np.ascontiguousarray(got, dtype=np.float32)
    ref = np.ascontiguousarray(ref, dtype=np.float32)
    assert got.shape == ref.shape
    bad = np.flatnonzero(got.view(np.uint32) != ref.view(np.uint32))
    assert bad.size == 0, f"{bad.size} results differ, first at {bad[0]}: {got.flat[bad[0]]!r} vs {ref.flat[bad[0]]!r}"


@pytest.mark.parametrize("t", [mm.F32, mm.F16])
def test_gemv_float_router_shape(ctx, orc, t):
    """f32 / f16 weights sum in math.matVecMul's order (math.zig:79-99: four
    lane accumulators, unfused products, ((a0 + a1) + a2) + a3, then the
    tail), so the router's scores are the CPU path's bits."""
    rng = np.random.default_rng(40 + t)
    raw = _weights(rng, t, 64, 2048)
    x = rng.standard_normal(2048).astype(np.float32)
    ref = orc.mat_vec_mul_unified(raw, t, x, 64, 2048)
    _bits_equal(ctx.mat_vec_mul(raw, t, x, 64, 2048), ref)


@pytest.mark.parametrize("t", [mm.F32, mm.F16])
@pytest.mark.parametrize("rows,cols", [(1, 1), (3, 5), (7, 33), (2, 2050), (5, 4099), (64, 6144), (2560, 512)])
def test_gemv_float_bit_exact_shapes(ctx, orc, t, rows, cols):
    """Tails of 1-3 columns, several product chunks, MLA's k_b / v_b expansion
    shape [2560 x 512] (inference.zig:539-544): bit-exact."""
    rng = np.random.default_rng(rows * 31 + cols + t)
    raw = _weights(rng, t, rows, cols)
    x = (rng.standard_normal(cols) * 3.0).astype(np.float32)
    _bits_equal(ctx.mat_vec_mul(raw, t, x, rows, cols), orc.mat_vec_mul_unified(raw, t, x, rows, cols))


@pytest.mark.parametrize("t,rows,cols", [
    (mm.Q8_0, 1, 32), (mm.Q8_0, 17, 96), (mm.Q8_0, 33, 40), (mm.Q8_0, 5, 1000),
    (mm.IQ2_XXS, 1, 256), (mm.IQ2_XXS, 17, 512), (mm.IQ2_XXS, 100, 768),
    (mm.F32, 3, 5), (mm.F16, 7, 33),
])
def test_gemv_ragged_shapes(ctx, orc, t, rows, cols):
    """Rows not a multiple of the 16-row tile; Q8_0 columns with a partial
    last block (the reference ignores columns >= in_dim)."""
    rng = np.random.default_rng(rows * 7 + cols)
    raw = _weights(rng, t, rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    ref = orc.mat_vec_mul_unified(raw, t, x, rows, cols)
    assert mm.max_abs_rel(ctx.mat_vec_mul(raw, t, x, rows, cols), ref) <= TOL_GEMV


def test_gemv_reference_kat_all_ones(ctx, orc):
    # qmm.zig:213-238 on the device: 4x64 all-127 blocks, d=f16(1/127), x=1 -> 64
    d, _ = orc.f32_to_f16(1.0 / 127.0)
    b = np.zeros((8, 34), np.uint8)
    b[:, 0:2] = np.array([d], np.uint16).view(np.uint8)
    b[:, 2:] = 127
    out = ctx.mat_vec_mul(b.reshape(-1), mm.Q8_0, np.ones(64, np.float32), 4, 64)
    assert np.all(np.abs(out - 64.0) <= 0.1)


def test_gemv_structured_layout_probe(ctx, orc):
    """One-hot activations select single columns: any mistake in the tile
    layout, the MFMA operand layout or the digit split shows up as a wrong
    column landing in a row."""
    rng = np.random.default_rng(77)
    rows, cols = 48, 512
    raw = _weights(rng, mm.IQ2_XXS, rows, cols)
    w = orc.dequantize(raw, orc.IQ2_XXS, rows * cols).reshape(rows, cols)
    for c in [0, 1, 7, 8, 31, 32, 100, 255, 256, 511]:
        x = np.zeros(cols, np.float32)
        x[c] = 1.0
        got = ctx.mat_vec_mul(raw, mm.IQ2_XXS, x, rows, cols)
        assert np.allclose(got, w[:, c], rtol=1e-4, atol=1e-7), f"column {c}"
    rawq = _weights(rng, mm.Q8_0, rows, cols)
    wq = orc.dequantize(rawq, orc.Q8_0, rows * cols).reshape(rows, cols)
    for c in [0, 5, 31, 32, 63, 64, 511]:
        x = np.zeros(cols, np.float32)
        x[c] = -2.5
        got = ctx.mat_vec_mul(rawq, mm.Q8_0, x, rows, cols)
        assert np.allclose(got, -2.5 * wq[:, c], rtol=1e-4, atol=1e-7), f"column {c}"


def test_gemv_batched_many_experts_one_launch(ctx, orc):
    """64 stacked expert matrices in one launch, distinct input per matrix."""
    rng = np.random.default_rng(8)
    rows, cols, E = 1536, 2048, 8
    raw = _weights(rng, mm.IQ2_XXS, rows, cols, E)
    w = ctx.upload(raw, mm.IQ2_XXS, rows, cols, E)
    x = rng.standard_normal((E, cols)).astype(np.float32)
    dx = mm.DeviceArray.from_numpy(ctx, x)
    dy = mm.DeviceArray(ctx, E * rows * 4)
    ctx.gemv_batched_dev(w, 0, E, dx, cols, dy, rows)
    ctx.synchronize()
    y = dy.to_numpy(np.float32, E * rows).reshape(E, rows)
    per = mm.tensor_bytes(mm.IQ2_XXS, rows, cols)
    for e in range(E):
        ref = orc.mat_vec_mul_unified(raw[e * per:(e + 1) * per], orc.IQ2_XXS, x[e], rows, cols)
        assert mm.max_abs_rel(y[e], ref) <= TOL_GEMV, f"expert {e}"
    # shared input vector (x_stride 0), sub-range of matrices
    ctx.gemv_batched_dev(w, 2, 3, dx, 0, dy, rows)
    ctx.synchronize()
    y = dy.to_numpy(np.float32, 3 * rows).reshape(3, rows)
    for i, e in enumerate(range(2, 5)):
        ref = orc.mat_vec_mul_unified(raw[e * per:(e + 1) * per], orc.IQ2_XXS, x[0], rows, cols)
        assert mm.max_abs_rel(y[i], ref) <= TOL_GEMV
    w.free()
    dx.free()
    dy.free()


def test_gemv_edge_values(ctx, orc):
    """Zero input, zero scales, huge and tiny activations, NaN/Inf poisoning."""
    rng = np.random.default_rng(9)
    rows, cols = 32, 512
    raw = _weights(rng, mm.IQ2_XXS, rows, cols)
    assert np.all(ctx.mat_vec_mul(raw, mm.IQ2_XXS, np.zeros(cols, np.float32), rows, cols) == 0.0)
    for scale in [1e30, 1e-30]:
        x = (rng.standard_normal(cols) * scale).astype(np.float32)
        ref = orc.mat_vec_mul_unified(raw, orc.IQ2_XXS, x, rows, cols)
        assert mm.max_abs_rel(ctx.mat_vec_mul(raw, mm.IQ2_XXS, x, rows, cols), ref) <= TOL_GEMV
    x = rng.standard_normal(cols).astype(np.float32)
    x[3] = np.inf
    got = ctx.mat_vec_mul(raw, mm.IQ2_XXS, x, rows, cols)
    ref = orc.mat_vec_mul_unified(raw, orc.IQ2_XXS, x, rows, cols)
    assert np.all(~np.isfinite(ref)) and np.all(~np.isfinite(got))
    zero_d = raw.reshape(-1, 66).copy()
    zero_d[:, 0:2] = 0
    assert np.all(ctx.mat_vec_mul(zero_d.reshape(-1), mm.IQ2_XXS, np.ones(cols, np.float32), rows, cols) == 0.0)


@pytest.mark.parametrize("t", [mm.Q8_0, mm.IQ2_XXS])
@pytest.mark.parametrize("rows,cols", [(1536, 2048), (2048, 1536)])
def test_qmm_batch64_config(ctx, orc, t, rows, cols):
    """Batched prefill QMM, batch 64, against the oracle's batchMatMulUnified."""
    rng = np.random.default_rng(rows + 5 * t)
    raw = _weights(rng, t, rows, cols)
    xin = rng.standard_normal((64, cols)).astype(np.float32)
    ref = orc.batch_mat_mul_unified(raw, t, xin, rows, 64, cols)
    got = ctx.batch_mat_mul(raw, t, xin, rows, 64, cols)
    err = mm.max_abs_rel(got, ref)
    print(f"qmm type={t} {rows}x{cols} max_abs_rel={err:.3e}")
    assert err <= TOL_QMM
    assert err <= TOL_GEMV   # the int8-digit MFMA path also meets the f32 bar


@pytest.mark.parametrize("t", [mm.F32, mm.F16])
@pytest.mark.parametrize("batch,rows,cols", [(5, 80, 320), (16, 64, 2048), (37, 200, 1024), (64, 64, 2048),
                                             (9, 48, 330), (17, 40, 4100)])
def test_float_weights_batched(ctx, orc, t, batch, rows, cols):
    """f32 / f16 weights times a batch (the router of a prefill call,
    batchMatMulUnified's f32 branch: one math.matVecMul per row,
    inference.zig:1256-1262): 16 vectors per workgroup share each row's
    loads, and every vector's sum keeps the single-vector order, so the
    results are the CPU path's bits for any batch."""
    rng = np.random.default_rng(batch * 7 + rows + t)
    raw = _weights(rng, t, rows, cols)
    xin = rng.standard_normal((batch, cols)).astype(np.float32)
    ref = orc.batch_mat_mul_unified(raw, t, xin, rows, batch, cols)
    got = ctx.batch_mat_mul(raw, t, xin, rows, batch, cols)
    _bits_equal(got, ref)


@pytest.mark.parametrize("batch", [1, 2, 7, 33, 100])
def test_qmm_ragged_batches_and_layouts(ctx, orc, batch):
    rng = np.random.default_rng(batch)
    rows, cols = 80, 320
    raw = _weights(rng, mm.Q8_0, rows, cols)
    xin = rng.standard_normal((batch, cols)).astype(np.float32)
    ref_mn = orc.matmul_q8_0(raw, xin, rows, batch, cols)          # [rows][batch], qmm.zig layout
    w = ctx.upload(raw, mm.Q8_0, rows, cols)
    dx = mm.DeviceArray.from_numpy(ctx, xin)
    dy = mm.DeviceArray(ctx, rows * batch * 4)
    for layout in (0, 1):
        ctx.qmm_dev(w, 0, dx, dy, batch, layout)
        ctx.synchronize()
        y = dy.to_numpy(np.float32, rows * batch)
        y = y.reshape(batch, rows).T if layout == 0 else y.reshape(rows, batch)
        assert mm.max_abs_rel(y, ref_mn) <= TOL_QMM
    w.free()
    dx.free()
    dy.free()


@pytest.mark.parametrize("cols", [256, 768, 1024, 1280, 1536, 1792, 2048, 2304])
def test_qmm_q8_every_k_split(ctx, orc, cols):
    """Q8_0 matmul over every K width the one-launch kernel splits its own
    way (units of 64 columns per 16-row tile: 4 -> one slice, 12 -> three
    one-step slices, 16 -> two, 20 -> five, 24 -> three two-step slices,
    28 -> seven, 32 -> four) and one past it (2304: the two-launch path),
    with a ragged batch and ragged rows, both output layouts, against the
    oracle's matMulQ8_0 (qmm.zig:58-138)."""
    rng = np.random.default_rng(cols)
    rows, batch = 100, 13
    raw = _weights(rng, mm.Q8_0, rows, cols)
    xin = rng.standard_normal((batch, cols)).astype(np.float32)
    ref_mn = orc.matmul_q8_0(raw, xin, rows, batch, cols)
    w = ctx.upload(raw, mm.Q8_0, rows, cols)
    dx = mm.DeviceArray.from_numpy(ctx, xin)
    dy = mm.DeviceArray(ctx, rows * batch * 4)
    try:
        for layout in (0, 1):
            ctx.qmm_dev(w, 0, dx, dy, batch, layout)
            ctx.synchronize()
            y = dy.to_numpy(np.float32, rows * batch)
            y = y.reshape(batch, rows).T if layout == 0 else y.reshape(rows, batch)
            assert mm.max_abs_rel(y, ref_mn) <= TOL_QMM, (cols, layout)
    finally:
        w.free()
        dx.free()
        dy.free()


def test_qmm_reference_kats(ctx, orc):
    # qmm.zig:142-173: 4x8x64 all-ones -> 64 +- 0.1
    d, _ = orc.f32_to_f16(1.0 / 127.0)
    b = np.zeros((8, 34), np.uint8)
    b[:, 0:2] = np.array([d], np.uint16).view(np.uint8)
    b[:, 2:] = 127
    out = ctx.batch_mat_mul(b.reshape(-1), mm.Q8_0, np.ones((8, 64), np.float32), 4, 8, 64)
    assert np.all(np.abs(out - 64.0) <= 0.1)
    # qmm.zig:175-211: batch result vs repeated GEMV within 0.01
    d, _ = orc.f32_to_f16(0.5 / 127.0)
    b = np.zeros((6, 34), np.uint8)
    b[:, 0:2] = np.array([d], np.uint16).view(np.uint8)
    b[:, 2:] = np.array([(i * 32 + j) % 127 for i in range(6) for j in range(32)], np.uint8).reshape(6, 32)
    raw = b.reshape(-1)
    bb = ((np.arange(5 * 64) % 7).astype(np.float32) * np.float32(0.3)).reshape(5, 64)
    out = ctx.batch_mat_mul(raw, mm.Q8_0, bb, 3, 5, 64)
    for ni in range(5):
        exp = ctx.mat_vec_mul(raw, mm.Q8_0, bb[ni], 3, 64)
        assert np.all(np.abs(exp - out[ni]) <= 0.01)


def test_seam_is_thread_safe(ctx, orc):
    """The reference re-enters the seam from 4 pool workers at once
    (inference.zig:934-971); 4 threads must get the same answers as 1."""
    rng = np.random.default_rng(10)
    rows, cols = 256, 1024
    raws = [_weights(rng, mm.IQ2_XXS, rows, cols) for _ in range(4)]
    xs = [rng.standard_normal(cols).astype(np.float32) for _ in range(4)]
    refs = [orc.mat_vec_mul_unified(r, orc.IQ2_XXS, x, rows, cols) for r, x in zip(raws, xs)]
    errs = []

    def work(i):
        for _ in range(20):
            y = ctx.mat_vec_mul(raws[i], mm.IQ2_XXS, xs[i], rows, cols)
            errs.append(mm.max_abs_rel(y, refs[i]))

    th = [threading.Thread(target=work, args=(i,)) for i in range(4)]
    for t in th:
        t.start()
    for t in th:
        t.join()
    assert len(errs) == 80 and max(errs) <= TOL_GEMV


@pytest.mark.parametrize("t", [mm.Q8_0, mm.IQ2_XXS])
@pytest.mark.parametrize("n_groups", [2, 3, 4])
def test_gemv_grouped_matches_separate(ctx, orc, t, n_groups):
    """mmhip_gemv_grouped_dev: weights of different shapes in one launch (the
    routed experts' gate/up [1536 x 2048] with a shared x, down [2048 x 1536]
    with one x each, and ragged shapes), against one mmhip_gemv_batched_dev per
    group (IQ2_XXS: bit for bit; Q8_0: f32 rounding) and the oracle."""
    rng = np.random.default_rng(700 + 10 * t + n_groups)
    shapes = [(1536, 2048, 5, True), (2048, 1536, 5, False), (100, 768, 3, False), (48, 2048, 2, True)][:n_groups]
    groups, sep, cases = [], [], []
    for rows, cols, n, shared in shapes:
        raw = mm.make_weight(rng, t, rows, cols, n + 1)
        w = ctx.upload(raw, t, rows, cols, n + 1)
        xs = rng.standard_normal((1 if shared else n, cols)).astype(np.float32)
        dx = mm.DeviceArray.from_numpy(ctx, xs)
        dy, dy2 = mm.DeviceArray(ctx, n * rows * 4), mm.DeviceArray(ctx, n * rows * 4)
        groups.append((w, 1, n, dx, 0 if shared else cols, dy, rows))  # matrices 1..n of the stack
        sep.append((w, dx, dy2, n, 0 if shared else cols, rows))
        cases.append((raw, xs, rows, cols, n, shared, dy, dy2, w))
    try:
        ctx.gemv_grouped_dev(groups)
        for w, dx, dy2, n, xs_, rows in sep:
            ctx.gemv_batched_dev(w, 1, n, dx, xs_, dy2, rows)
        ctx.synchronize()
        per_mat = mm.tensor_bytes(t, shapes[0][0], shapes[0][1])
        for raw, xs, rows, cols, n, shared, dy, dy2, w in cases:
            got = dy.to_numpy(np.float32, n * rows).reshape(n, rows)
            ref = dy2.to_numpy(np.float32, n * rows).reshape(n, rows)
            if t == mm.IQ2_XXS:
                _bits_equal(got, ref)
            per_mat = mm.tensor_bytes(t, rows, cols)
            for i in range(n):
                x = xs[0 if shared else i]
                cpu = orc.mat_vec_mul_unified(raw[(i + 1) * per_mat:(i + 2) * per_mat], t, x, rows, cols)
                assert mm.max_abs_rel(got[i], cpu) <= TOL_GEMV
    finally:
        for raw, xs, rows, cols, n, shared, dy, dy2, w in cases:
            dy.free()
            dy2.free()
            w.free()
        for g in groups:
            g[3].free()


def test_gemv_grouped_rejects_bad_groups(ctx):
    rng = np.random.default_rng(760)
    wq = ctx.upload(mm.make_weight(rng, mm.Q8_0, 16, 256), mm.Q8_0, 16, 256)
    wi = ctx.upload(mm.make_weight(rng, mm.IQ2_XXS, 16, 256), mm.IQ2_XXS, 16, 256)
    x, y = mm.DeviceArray(ctx, 256 * 4), mm.DeviceArray(ctx, 16 * 4)
    try:
        with pytest.raises(mm.MmhipError):
            ctx.gemv_grouped_dev([(wq, 0, 1, x, 0, y, 16), (wi, 0, 1, x, 0, y, 16)])  # two types
        with pytest.raises(mm.MmhipError):
            ctx.gemv_grouped_dev([(wq, 0, 2, x, 0, y, 16)])  # past the weight's one matrix
        with pytest.raises(mm.MmhipError):
            ctx.gemv_grouped_dev([(wq, 0, 1, x, 0, y, 16)] * 5)  # more than MMHIP_GEMV_MAX_GROUPS
    finally:
        for a in (wq, wi, x, y):
            a.free()


def test_weight_over_2gib_per_matrix_is_rejected(ctx):
    # 2^21 rows of 1024 Q8_0 columns repack to exactly 2 GiB of records; the
    # kernels address one matrix with 32-bit offsets, so the upload refuses it
    # before allocating. The source is a full-size zero buffer (calloc, pages
    # untouched) so that a missing check would still read only valid memory.
    rows, cols = 1 << 21, 1024
    raw = np.zeros(rows * (cols // 32) * 34, np.uint8)
    with pytest.raises(mm.MmhipError) as e:
        ctx.upload(raw, mm.Q8_0, rows, cols)
    assert e.value.code == mm.ERR_UNSUPPORTED


@pytest.mark.parametrize("t", [mm.IQ2_XXS, mm.Q8_0])
def test_headline_step_shape_matches_oracle(ctx, orc, t):
    """The benchmark's headline launch exactly as it is measured: one
    mmhip_gemv_grouped_dev call over 64 distinct [1536 x 2048] matrices with a
    shared x and 64 distinct [2048 x 1536] matrices with one x each (the
    routed experts' gate/up and down of a GLM-4.7-Flash layer,
    inference.zig:1171-1185). The launcher gives each workgroup 48 (gate
    shape) or 64 (down shape) row tiles, which fills all of its LDS partial
    slots. Every matrix against the oracle's matVecMulUnified within 1e-3;
    IQ2_XXS also bit for bit against one mmhip_gemv_batched_dev launch per
    matrix."""
    E, H, I = 64, 2048, 1536
    rng = np.random.default_rng(4100 + t)
    raw_g = mm.make_weight(rng, t, I, H, E)
    raw_d = mm.make_weight(rng, t, H, I, E)
    x = rng.standard_normal(H).astype(np.float32)
    xd = rng.standard_normal((E, I)).astype(np.float32)
    wg, wd = ctx.upload(raw_g, t, I, H, E), ctx.upload(raw_d, t, H, I, E)
    dx, dxd = mm.DeviceArray.from_numpy(ctx, x), mm.DeviceArray.from_numpy(ctx, xd)
    yg, yd = mm.DeviceArray(ctx, E * I * 4), mm.DeviceArray(ctx, E * H * 4)
    yg1, yd1 = mm.DeviceArray(ctx, I * 4), mm.DeviceArray(ctx, H * 4)
    try:
        ctx.gemv_grouped_dev([(wg, 0, E, dx, 0, yg, I), (wd, 0, E, dxd, I, yd, H)])
        ctx.synchronize()
        got_g = yg.to_numpy(np.float32, E * I).reshape(E, I)
        got_d = yd.to_numpy(np.float32, E * H).reshape(E, H)
        pg, pd = mm.tensor_bytes(t, I, H), mm.tensor_bytes(t, H, I)
        worst = 0.0
        for e in range(E):
            rg = orc.mat_vec_mul_unified(raw_g[e * pg:(e + 1) * pg], t, x, I, H)
            rd = orc.mat_vec_mul_unified(raw_d[e * pd:(e + 1) * pd], t, xd[e], H, I)
            worst = max(worst, mm.max_abs_rel(got_g[e], rg), mm.max_abs_rel(got_d[e], rd))
        assert worst <= TOL_GEMV, worst
        if t == mm.IQ2_XXS:
            for e in (0, 1, 17, 40, 63):
                ctx.gemv_batched_dev(wg, e, 1, dx, 0, yg1, 0)
                ctx.synchronize()
                _bits_equal(got_g[e], yg1.to_numpy(np.float32, I))
            # Down shape: each single-matrix launch takes its own x row.
            for e in (0, 5, 63):
                xe = mm.DeviceArray.from_numpy(ctx, np.ascontiguousarray(xd[e]))
                try:
                    ctx.gemv_batched_dev(wd, e, 1, xe, 0, yd1, 0)
                    ctx.synchronize()
                    _bits_equal(got_d[e], yd1.to_numpy(np.float32, H))
                finally:
                    xe.free()
    finally:
        for a in (wg, wd, dx, dxd, yg, yd, yg1, yd1):
            a.free()


_SHAPE_CHILD = r'''
import sys
import numpy as np
import mmhip as mm
out = sys.argv[1]
ctx = mm.Context(0)
rng = np.random.default_rng(880)
res = {}
# Two segments in one launch (a shared x, one x per matrix), as the decode step runs them.
g_raw = mm.make_weight(rng, mm.IQ2_XXS, 1536, 2048, 6)
d_raw = mm.make_weight(rng, mm.IQ2_XXS, 2048, 1536, 6)
gw, dw = ctx.upload(g_raw, mm.IQ2_XXS, 1536, 2048, 6), ctx.upload(d_raw, mm.IQ2_XXS, 2048, 1536, 6)
x = mm.DeviceArray.from_numpy(ctx, rng.standard_normal(2048).astype(np.float32))
xd = mm.DeviceArray.from_numpy(ctx, rng.standard_normal((6, 1536)).astype(np.float32))
yg, yd = mm.DeviceArray(ctx, 6 * 1536 * 4), mm.DeviceArray(ctx, 6 * 2048 * 4)
ctx.gemv_grouped_dev([(gw, 0, 6, x, 0, yg, 1536), (dw, 0, 6, xd, 1536, yd, 2048)])
ctx.synchronize()
res["gate"], res["down"] = yg.to_numpy(np.float32, 6 * 1536), yd.to_numpy(np.float32, 6 * 2048)
# One matrix per call: a single tile per workgroup, and a K of several activation chunks.
for name, rows, cols in (("one", 2048, 1536), ("wide", 100, 5120)):
    raw = mm.make_weight(rng, mm.IQ2_XXS, rows, cols)
    res[name] = ctx.mat_vec_mul(raw, mm.IQ2_XXS, rng.standard_normal(cols).astype(np.float32), rows, cols)
np.savez(out, **res)
'''


def test_iq2_workgroup_shapes_give_the_same_bits(tmp_path):
    """The IQ2_XXS decode GEMV's two workgroup shapes (two 768-thread
    workgroups per CU, the default, and one 1024-thread workgroup,
    MMHIP_IQ2_PAIR=0) sum every row in the same order, so they must give the
    same bits. The shape is chosen once per process, so each runs in a child
    process on the same seeded inputs."""
    import os
    import subprocess
    import sys
    env_base = dict(os.environ)
    env_base["PYTHONPATH"] = os.pathsep.join([os.path.dirname(mm.__file__), env_base.get("PYTHONPATH", "")])
    outs = {}
    for pair in ("1", "0"):
        env = dict(env_base, MMHIP_IQ2_PAIR=pair)
        out = tmp_path / f"shape_{pair}.npz"
        r = subprocess.run([sys.executable, "-c", _SHAPE_CHILD, str(out)], env=env, capture_output=True, text=True,
                           timeout=300)
        assert r.returncode == 0, r.stderr[-2000:]
        outs[pair] = np.load(out)
    for k in ("gate", "down", "one", "wide"):
        a, b = outs["1"][k], outs["0"][k]
        assert a.shape == b.shape and np.all(np.isfinite(a))
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), k
