"""The MLA attention projections of the GLM-4.7-Flash shape on the same
kernels (inference.zig:467-489 decode, 684-706 batch, 521-568 k_b / v_b),
against the oracle's matVecMulUnified / batchMatMulUnified / math.matVecMul.
Dimensions: hidden 2048, q_lora 768, kv_lora 512, 20 heads, qk_nope 128,
qk_rope 64, v_head 128 (model.zig:80-90 defaults; tests/integration.zig:69-74)."""
import numpy as np
import pytest

import mmhip as mm

pytestmark = pytest.mark.gpu

H, QL, KVL, NH, NOPE, ROPE, VH = 2048, 768, 512, 20, 128, 64, 128
PROJ = {  # name: (out_dim, in_dim)
    "q_a": (QL, H),
    "q_b": (NH * (NOPE + ROPE), QL),
    "kv_a": (KVL + ROPE, H),
    "o_proj": (H, NH * VH),
}
TOL_GEMV, TOL_QMM = 1e-3, 1e-2


@pytest.mark.parametrize("t", [mm.Q8_0, mm.IQ2_XXS])
@pytest.mark.parametrize("name", list(PROJ))
def test_mla_projection_decode(ctx, orc, t, name):
    out_dim, in_dim = PROJ[name]
    rng = np.random.default_rng(sum(map(ord, name)) * 31 + t)
    raw = mm.make_weight(rng, t, out_dim, in_dim)
    x = rng.standard_normal(in_dim).astype(np.float32)
    ref = orc.mat_vec_mul_unified(raw, t, x, out_dim, in_dim)
    assert mm.max_abs_rel(ctx.mat_vec_mul(raw, t, x, out_dim, in_dim), ref) <= TOL_GEMV


@pytest.mark.parametrize("t", [mm.Q8_0, mm.IQ2_XXS])
@pytest.mark.parametrize("name", ["q_a", "kv_a", "o_proj"])
def test_mla_projection_batch(ctx, orc, t, name):
    """mlaAttentionBatch's projections (batchMatMulUnified) at batch 64."""
    out_dim, in_dim = PROJ[name]
    rng = np.random.default_rng(sum(map(ord, name)) * 37 + t + 64)
    raw = mm.make_weight(rng, t, out_dim, in_dim)
    xin = rng.standard_normal((64, in_dim)).astype(np.float32)
    ref = orc.batch_mat_mul_unified(raw, t, xin, out_dim, 64, in_dim)
    got = ctx.batch_mat_mul(raw, t, xin, out_dim, 64, in_dim)
    assert mm.max_abs_rel(got, ref) <= TOL_QMM


@pytest.mark.parametrize("n_pos", [1, 37, 300])
def test_mla_kv_expansion_f32(ctx, orc, n_pos):
    """k_b / v_b: f32 [2560 x 512] (dequantized once, inference.zig:528-535)
    applied to every cached position's kv_comp (the expansion loop, 557-566):
    one batched float GEMV over the positions."""
    rng = np.random.default_rng(n_pos)
    w = rng.normal(0.0, 0.05, (NH * NOPE, KVL)).astype(np.float32)
    kv = rng.standard_normal((n_pos, KVL)).astype(np.float32)
    ref = np.stack([orc.mat_vec_mul_unified(w.view(np.uint8).reshape(-1), mm.F32, kv[p], NH * NOPE, KVL)
                    for p in range(n_pos)])
    got = ctx.batch_mat_mul(w.view(np.uint8).reshape(-1), mm.F32, kv, NH * NOPE, n_pos, KVL)
    assert mm.max_abs_rel(got, ref) <= TOL_GEMV


@pytest.mark.parametrize("fmt", [mm.Q8_0, mm.IQ2_XXS])
def test_fused_q_a_kv_a(ctx, orc, fmt):
    """q_a and kv_a read the same hidden vector, so their raw rows stacked into
    one [1344 x 2048] weight give both projections in one launch: the same
    bits as the two separate GEMVs, and the oracle's to 1e-3."""
    rng = np.random.default_rng(500 + fmt)
    qa, kva = mm.make_weight(rng, fmt, 768, 2048), mm.make_weight(rng, fmt, 576, 2048)
    qkv = np.concatenate([qa, kva])
    x = rng.standard_normal(2048).astype(np.float32)
    fused = ctx.mat_vec_mul(qkv, fmt, x, 768 + 576, 2048)
    assert np.array_equal(fused[:768].view(np.uint32), ctx.mat_vec_mul(qa, fmt, x, 768, 2048).view(np.uint32))
    assert np.array_equal(fused[768:].view(np.uint32), ctx.mat_vec_mul(kva, fmt, x, 576, 2048).view(np.uint32))
    ref = orc.mat_vec_mul_unified(qkv, fmt, x, 768 + 576, 2048)
    assert mm.max_abs_rel(fused, ref) <= TOL_GEMV
