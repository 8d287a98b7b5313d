"""Parity on realistic activations at the GLM-4.7-Flash shape.

The kernels hold activations as 16-bit block fixed point (one scale per 32
columns in the decode GEMV, per 256 columns in the grouped prefill and the
IQ2_XXS QMM), so a block's small entries lose resolution next to a large one.
These tests feed what real hidden states look like instead of N(0, 1):

- student_t: heavy tails, Student-t with 2 degrees of freedom;
- outliers: N(0, 1) with four fixed channels at +300, +1000, +3000 and -3000
  (the massive-activation channels of transformer residual streams).

Each case is compared with the oracle (the reference CPU path) on the same
inputs: max-abs-rel = max|y - r| / max|r| against the bar of the path (1e-3
for the f32-accumulating GEMV and MoE paths, 1e-2 for the batched QMM), and
the 99.9th percentile of |y - r| / max(|r|, 1e-6 max|r|) is printed beside it
(run pytest with -s to see the table).
"""
import numpy as np
import pytest

import mmhip as mm

pytestmark = pytest.mark.gpu

H, I, E = 2048, 1536, 64
OUTLIER_CH = (17, 613, 1290, 2001)
OUTLIER_VAL = (300.0, 1000.0, 3000.0, -3000.0)


def acts(kind, rng, n, cols):
    if kind == "student_t":
        return rng.standard_t(2.0, size=(n, cols)).astype(np.float32)
    x = rng.standard_normal((n, cols)).astype(np.float32)
    for c, v in zip(OUTLIER_CH, OUTLIER_VAL):
        if c < cols:
            x[:, c] = np.float32(v) * (1.0 + 0.01 * rng.standard_normal(n)).astype(np.float32)
    return x


def errors(got, ref):
    got = np.asarray(got, np.float64).reshape(-1)
    ref = np.asarray(ref, np.float64).reshape(-1)
    scale = np.max(np.abs(ref))
    rel = np.abs(got - ref) / np.maximum(np.abs(ref), 1e-6 * scale)
    return mm.max_abs_rel(got, ref), float(np.percentile(rel, 99.9))


@pytest.mark.parametrize("kind", ["student_t", "outliers"])
@pytest.mark.parametrize("t", [mm.IQ2_XXS, mm.Q8_0])
@pytest.mark.parametrize("rows,cols", [(1536, 2048), (2048, 1536)])
def test_decode_gemv_realistic(ctx, orc, kind, t, rows, cols):
    rng = np.random.default_rng(1000 + rows + t + (kind == "outliers"))
    raw = mm.make_weight(rng, t, rows, cols)
    x = acts(kind, rng, 1, cols)[0]
    got = ctx.mat_vec_mul(raw, t, x, rows, cols)
    mar, p999 = errors(got, orc.mat_vec_mul_unified(raw, t, x, rows, cols))
    print(f"\ndecode GEMV {kind:9s} type {t:2d} [{rows}x{cols}]: max-abs-rel {mar:.2e}  p99.9 {p999:.2e}")
    assert mar <= 1e-3


@pytest.mark.parametrize("kind", ["student_t", "outliers"])
@pytest.mark.parametrize("t", [mm.Q8_0, mm.IQ2_XXS])
def test_batched_qmm_realistic(ctx, orc, kind, t):
    """X[64 x 2048] through batchMatMulUnified (Q8_0: matMulQ8_0's order,
    qmm.zig:58-138; IQ2_XXS: dequantize + f32 GEMV per row)."""
    rng = np.random.default_rng(1100 + t + (kind == "outliers"))
    rows, cols, batch = 1536, 2048, 64
    raw = mm.make_weight(rng, t, rows, cols)
    X = acts(kind, rng, batch, cols)
    got = ctx.batch_mat_mul(raw, t, X, rows, batch, cols)
    mar, p999 = errors(got, orc.batch_mat_mul_unified(raw, t, X, rows, batch, cols))
    print(f"\nbatched QMM {kind:9s} type {t:2d} [64x2048]x[1536x2048]^T: max-abs-rel {mar:.2e}  p99.9 {p999:.2e}")
    assert mar <= 1e-2


@pytest.fixture(scope="module")
def glm_layer(ctx, orc):
    rng = np.random.default_rng(1200)
    kw = dict(hidden=H, inter=I, n_experts=E, expert_type=mm.IQ2_XXS,
              router=rng.normal(0.0, 0.02, (E, H)).astype(np.float32),
              gate=mm.make_iq2_xxs(rng, I, H, E), up=mm.make_iq2_xxs(rng, I, H, E),
              down=mm.make_iq2_xxs(rng, H, I, E),
              shared=(mm.make_iq2_xxs(rng, I, H), mm.make_iq2_xxs(rng, I, H), mm.make_iq2_xxs(rng, H, I)),
              shared_inter=I)
    gpu = mm.MoeLayer(ctx, **kw)
    cpu = orc.Moe(**kw)
    pool = orc.Pool(4)
    yield gpu, cpu, pool
    pool.close()
    gpu.free()


@pytest.mark.parametrize("kind", ["student_t", "outliers"])
@pytest.mark.parametrize("t", [1, 64])
def test_moe_layer_realistic(glm_layer, kind, t):
    """One MoE layer (64 IQ2_XXS experts of width 1536, top-4 + shared),
    decode (t = 1) and grouped prefill (t = 64): route ids exact, outputs at
    the f32 bar."""
    gpu, cpu, pool = glm_layer
    rng = np.random.default_rng(1300 + t + (kind == "outliers"))
    h = acts(kind, rng, t, H)
    out_g, ids_g, w_g = gpu.ffn(h)
    out_c, ids_c, w_c = cpu.ffn(h, pool=pool)
    np.testing.assert_array_equal(ids_g, ids_c)
    np.testing.assert_allclose(w_g, w_c, rtol=1e-6, atol=1e-7)
    mar, p999 = errors(out_g, out_c)
    print(f"\nMoE layer {kind:9s} tokens {t:2d}: max-abs-rel {mar:.2e}  p99.9 {p999:.2e}")
    assert mar <= 1e-3
