"""Committed golden vectors (tests/golden/golden.npz, written by
tests/golden/make_golden.py from the oracle): the oracle still reproduces
them bit for bit (CPU), and the HIP path matches them (GPU: dequantisation
bit-exact, products within max-abs-rel 1e-3, MoE route ids exact)."""
import os

import numpy as np
import pytest

import mmhip as mm

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "golden.npz")


@pytest.fixture(scope="module")
def g():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _moe_kw(g, orc_or_mm):
    return dict(hidden=256, inter=256, n_experts=8, expert_type=orc_or_mm.IQ2_XXS, router=g["moe_router"],
                gate=g["moe_gate"], up=g["moe_up"], down=g["moe_down"],
                shared=(g["moe_shared_gate"], g["moe_shared_up"], g["moe_shared_down"]), shared_inter=256)


def test_oracle_reproduces_golden(orc, g):
    assert np.array_equal(orc.dequantize(g["iq2_blocks"], orc.IQ2_XXS, 2048), g["iq2_blocks_deq"])
    assert np.array_equal(orc.dequantize(g["q8_blocks"], orc.Q8_0, 256), g["q8_blocks_deq"])
    assert np.array_equal(orc.mat_vec_mul_unified(g["gemv_iq2_w"], orc.IQ2_XXS, g["gemv_iq2_x"], 64, 256),
                          g["gemv_iq2_y"])
    assert np.array_equal(orc.matvec_q8_0(g["gemv_q8_w"], g["gemv_q8_x"], 32, 64), g["gemv_q8_y"])
    assert np.array_equal(orc.matmul_q8_0(g["qmm_w"], g["qmm_x"], 8, 4, 64), g["qmm_c"])
    out, ids, w = orc.Moe(**_moe_kw(g, orc)).ffn(g["moe_hidden"])
    assert np.array_equal(ids, g["moe_ids"]) and np.array_equal(w, g["moe_w"]) and np.array_equal(out, g["moe_out"])


def test_golden_shapes(g):
    assert g["iq2_blocks"].size == 8 * 66 and g["q8_blocks"].size == 8 * 34
    assert g["moe_ids"].shape == (3, 4) and g["qmm_c"].shape == (8, 4)


@pytest.mark.gpu
def test_hip_path_matches_golden(ctx, g):
    assert np.array_equal(ctx.dequantize(g["iq2_blocks"], mm.IQ2_XXS, 2048), g["iq2_blocks_deq"])
    assert np.array_equal(ctx.dequantize(g["q8_blocks"], mm.Q8_0, 256), g["q8_blocks_deq"])
    y = ctx.mat_vec_mul(g["gemv_iq2_w"], mm.IQ2_XXS, g["gemv_iq2_x"], 64, 256)
    assert mm.max_abs_rel(y, g["gemv_iq2_y"]) < 1e-3
    y = ctx.mat_vec_mul(g["gemv_q8_w"], mm.Q8_0, g["gemv_q8_x"], 32, 64)
    assert mm.max_abs_rel(y, g["gemv_q8_y"]) < 1e-3
    c = ctx.batch_mat_mul(g["qmm_w"], mm.Q8_0, g["qmm_x"], 8, 4, 64)   # [batch][out_dim]
    assert mm.max_abs_rel(c.T, g["qmm_c"]) < 1e-3
    layer = mm.MoeLayer(ctx, **_moe_kw(g, mm))
    try:
        out, ids, w = layer.ffn(g["moe_hidden"])
        np.testing.assert_array_equal(ids, g["moe_ids"])
        np.testing.assert_allclose(w, g["moe_w"], rtol=1e-6, atol=1e-7)
        assert mm.max_abs_rel(out, g["moe_out"]) < 1e-3
    finally:
        layer.free()
