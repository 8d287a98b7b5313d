"""Worst-case error of the activation format (16-bit block fixed point: two
int8 digits and one f32 scale per block of B columns) on the device, against
an exact product of the reference's dequantised weights
(dequant.zig:316-390; the GEMV / QMM themselves: qmm.zig:13-138,
inference.zig:1200-1264).

Per element the quantiser keeps |x - s q| < 1.6e-5 m (m = the block's max
|x|, s = m / 32512, q = rint(x / s) clamped to +-32512), so a dot product
is off by at most 1.6e-5 * sum_b m_b * sum_{i in b} |w_i| from the exact
product of the dequantised weights, plus the f32 rounding of the
per-block scaling and the sum over blocks (allowed here as 1e-5 of
sum |w_i x_i|, generous for 8..64 block terms). The activations are built
to stress that bound: a few entries 1e4 times the rest in some blocks,
blocks of zeros, blocks below 1e-30, and mixed signs. B is 32 for the
decode GEMVs and the Q8_0 matmul, 256 for the IQ2_XXS matmul.
"""
import numpy as np
import pytest

import mmhip as mm

pytestmark = pytest.mark.gpu

Q_REL = 1.6e-5   # per-element bound, relative to the block's max |x|
F32_SLACK = 1e-5  # f32 scaling and block sums, relative to sum |w_i x_i|


def _adversarial_x(rng, n, cols):
    x = rng.standard_normal((n, cols)).astype(np.float64)
    for r in range(n):
        nb = cols // 32
        blocks = rng.permutation(nb)
        for b in blocks[: nb // 4]:  # an outlier 1e4 times the rest
            x[r, b * 32 + rng.integers(32)] = rng.choice([-1.0, 1.0]) * 1e4
        for b in blocks[nb // 4: nb // 4 + 2]:
            x[r, b * 32:(b + 1) * 32] = 0.0
        for b in blocks[nb // 4 + 2: nb // 4 + 4]:
            x[r, b * 32:(b + 1) * 32] *= 1e-31
    return x.astype(np.float32)


def _bound(w, x, block):
    """Per output row: the format's bound plus the f32 slack."""
    w64, x64 = np.abs(w.astype(np.float64)), x.astype(np.float64)
    cols = x.shape[-1]
    m = np.abs(x64).reshape(x.shape[0], cols // block, block).max(axis=2)   # [n][blocks]
    wb = w64.reshape(w.shape[0], cols // block, block).sum(axis=2)          # [rows][blocks]
    return Q_REL * (m @ wb.T) + F32_SLACK * (np.abs(x64) @ w64.T)          # [n][rows]


@pytest.mark.parametrize("fmt", [mm.Q8_0, mm.IQ2_XXS])
def test_gemv_within_format_bound(ctx, orc, fmt):
    rng = np.random.default_rng(400 + fmt)
    rows, cols = 256, 2048
    raw = mm.make_weight(rng, fmt, rows, cols)
    w = orc.dequantize(raw, fmt, rows * cols).reshape(rows, cols)
    x = _adversarial_x(rng, 3, cols)
    exact = x.astype(np.float64) @ w.astype(np.float64).T
    bound = _bound(w, x, 32)
    for r in range(x.shape[0]):
        y = ctx.mat_vec_mul(raw, fmt, x[r], rows, cols).astype(np.float64)
        err = np.abs(y - exact[r])
        worst = float((err / bound[r]).max())
        print(f"gemv fmt={fmt} vector {r}: error / bound at most {worst:.3f}")
        assert np.all(err <= bound[r])


@pytest.mark.parametrize("fmt,block", [(mm.Q8_0, 32), (mm.IQ2_XXS, 256)])
def test_qmm_within_format_bound(ctx, orc, fmt, block):
    rng = np.random.default_rng(500 + fmt)
    rows, cols, batch = 256, 2048, 5
    raw = mm.make_weight(rng, fmt, rows, cols)
    w = orc.dequantize(raw, fmt, rows * cols).reshape(rows, cols)
    x = _adversarial_x(rng, batch, cols)
    exact = x.astype(np.float64) @ w.astype(np.float64).T
    bound = _bound(w, x, block)
    y = ctx.batch_mat_mul(raw, fmt, x, rows, batch, cols).astype(np.float64)
    err = np.abs(y - exact)
    print(f"qmm fmt={fmt}: error / bound at most {float((err / bound).max()):.3f}")
    assert np.all(err <= bound)
