"""Writes tests/golden/golden.npz: small seeded cases and the oracle's outputs.

Run from the repository root after `make -C oracle`:
    python tests/golden/make_golden.py
Inputs are raw GGUF bytes (Q8_0 / IQ2_XXS blocks, f32 vectors); outputs come
from the oracle (the C restatement of the reference CPU path). The file holds
plain arrays only (numpy .npz, no pickled objects).
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "mobile-moe.zig_amd", "python"))

import oracle as orc  # noqa: E402
import mmhip as mm  # noqa: E402


def build():
    rng = np.random.default_rng(0x5EED)
    g = {}
    # 8 IQ2_XXS superblocks (one row of 2048) and 8 Q8_0 blocks (one row of 256).
    g["iq2_blocks"] = mm.make_iq2_xxs(rng, 1, 2048)
    g["iq2_blocks_deq"] = orc.dequantize(g["iq2_blocks"], orc.IQ2_XXS, 2048)
    g["q8_blocks"] = mm.make_q8_0(rng, 1, 256)
    g["q8_blocks_deq"] = orc.dequantize(g["q8_blocks"], orc.Q8_0, 256)
    # IQ2_XXS GEMV 64 x 256 (matVecMulUnified's dequantize + f32 GEMV).
    g["gemv_iq2_w"] = mm.make_iq2_xxs(rng, 64, 256)
    g["gemv_iq2_x"] = rng.standard_normal(256).astype(np.float32)
    g["gemv_iq2_y"] = orc.mat_vec_mul_unified(g["gemv_iq2_w"], orc.IQ2_XXS, g["gemv_iq2_x"], 64, 256)
    # Q8_0 GEMV 32 x 64 (qmm.matVecMulQ8_0).
    g["gemv_q8_w"] = mm.make_q8_0(rng, 32, 64)
    g["gemv_q8_x"] = rng.standard_normal(64).astype(np.float32)
    g["gemv_q8_y"] = orc.matvec_q8_0(g["gemv_q8_w"], g["gemv_q8_x"], 32, 64)
    # Q8_0 QMM: W [8 x 64], X [4 x 64] -> C [8][4] (qmm.matMulQ8_0's layout).
    g["qmm_w"] = mm.make_q8_0(rng, 8, 64)
    g["qmm_x"] = rng.standard_normal((4, 64)).astype(np.float32)
    g["qmm_c"] = orc.matmul_q8_0(g["qmm_w"], g["qmm_x"], 8, 4, 64)
    # Tiny MoE layer: hidden 256, 8 IQ2_XXS experts of width 256, top-4 +
    # shared expert, f32 router; 3 tokens.
    H, I, E = 256, 256, 8
    g["moe_router"] = rng.normal(0.0, 0.05, (E, H)).astype(np.float32)
    g["moe_gate"] = mm.make_iq2_xxs(rng, I, H, E)
    g["moe_up"] = mm.make_iq2_xxs(rng, I, H, E)
    g["moe_down"] = mm.make_iq2_xxs(rng, H, I, E)
    g["moe_shared_gate"] = mm.make_iq2_xxs(rng, I, H)
    g["moe_shared_up"] = mm.make_iq2_xxs(rng, I, H)
    g["moe_shared_down"] = mm.make_iq2_xxs(rng, H, I)
    g["moe_hidden"] = rng.standard_normal((3, H)).astype(np.float32)
    moe = orc.Moe(hidden=H, inter=I, n_experts=E, expert_type=orc.IQ2_XXS, router=g["moe_router"],
                  gate=g["moe_gate"], up=g["moe_up"], down=g["moe_down"],
                  shared=(g["moe_shared_gate"], g["moe_shared_up"], g["moe_shared_down"]), shared_inter=I)
    out, ids, w = moe.ffn(g["moe_hidden"])
    g["moe_out"], g["moe_ids"], g["moe_w"] = out, ids, w
    return g


if __name__ == "__main__":
    g = build()
    np.savez(os.path.join(HERE, "golden.npz"), **g)
    print("wrote", os.path.join(HERE, "golden.npz"), sum(v.nbytes for v in g.values()), "bytes")
