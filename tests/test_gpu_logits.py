"""Output projection and greedy sampling on the GPU (computeLogits,
inference.zig:1189-1197; sampleGreedy, 376-386) against the oracle."""
import numpy as np
import pytest

import mmhip as mm

pytestmark = pytest.mark.gpu

VOCAB, HIDDEN = 154880, 2048  # deepseek2.vocab_size default (model.zig:115), hidden 2048


def _greedy_dev(ctx, logits, offset_floats=0):
    buf = np.zeros(logits.size + offset_floats, dtype=np.float32)
    buf[offset_floats:] = logits
    d = mm.DeviceArray.from_numpy(ctx, buf)
    o = mm.DeviceArray(ctx, 4)
    try:
        mm.check(ctx.lib.mmhip_argmax_dev(ctx.handle, o.ptr, d.ptr + 4 * offset_floats, logits.size), "argmax_dev")
        ctx.synchronize()
        return int(o.to_numpy(np.uint32, 1)[0])
    finally:
        d.free(); o.free()


@pytest.mark.parametrize("case", ["ties", "neg_zero", "pos_zero_first", "nan_first", "nan_later", "all_neg_inf",
                                  "all_equal", "single", "odd_tail"])
def test_sample_greedy_cases(ctx, orc, case):
    f = np.float32
    x = {
        "ties": np.array([1, 3, 3, 2], f),
        "neg_zero": np.array([-0.0, 0.0], f),
        "pos_zero_first": np.array([0.0, -0.0, -1.0], f),
        "nan_first": np.array([np.nan, 5, 9], f),
        "nan_later": np.array([1, np.nan, 0.5, 2, np.nan], f),
        "all_neg_inf": np.array([-np.inf, np.nan, -np.inf], f),
        "all_equal": np.full(4103, 2.5, f),
        "single": np.array([4.0], f),
        "odd_tail": np.concatenate([np.zeros(5000, f), np.array([7.0, 7.0], f)]),
    }[case]
    want = orc.sample_greedy(x)
    assert ctx.sample_greedy(x) == want
    assert _greedy_dev(ctx, x, offset_floats=1) == want  # 4-byte aligned only: the per-value loads


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_sample_greedy_vocab_random(ctx, orc, seed):
    rng = np.random.default_rng(seed)
    x = rng.integers(-1000, 1000, VOCAB).astype(np.float32)  # many exact ties at the maximum
    x[rng.integers(0, VOCAB, 50)] = np.nan
    assert ctx.sample_greedy(x) == orc.sample_greedy(x)
    x = rng.standard_normal(VOCAB).astype(np.float32)
    assert ctx.sample_greedy(x) == orc.sample_greedy(x) == int(np.argmax(x))


@pytest.mark.parametrize("t", [mm.Q8_0, mm.IQ2_XXS])
def test_output_projection_and_greedy(ctx, orc, t):
    """computeLogits at the real shape: [154880 x 2048] weight of the GGUF's
    type, f32 accumulation (1e-3 max-abs-rel), then sampleGreedy on the
    device logits."""
    rng = np.random.default_rng(20 + t)
    raw = mm.make_weight(rng, t, VOCAB, HIDDEN)
    h = rng.standard_normal(HIDDEN).astype(np.float32)
    ref = orc.mat_vec_mul_unified(raw, t, h, VOCAB, HIDDEN)
    w = ctx.upload(raw, t, VOCAB, HIDDEN)
    dx = mm.DeviceArray.from_numpy(ctx, h)
    dy = mm.DeviceArray(ctx, VOCAB * 4)
    do = mm.DeviceArray(ctx, 4)
    try:
        ctx.gemv_batched_dev(w, 0, 1, dx, 0, dy, 0)
        ctx.argmax_dev(do, dy, VOCAB)
        ctx.synchronize()
        logits = dy.to_numpy(np.float32, VOCAB)
        tok = int(do.to_numpy(np.uint32, 1)[0])
        assert mm.max_abs_rel(logits, ref) <= 1e-3
        assert tok == orc.sample_greedy(logits)
        assert ref[tok] >= ref.max() - 1e-3 * np.abs(ref).max()
    finally:
        w.free(); dx.free(); dy.free(); do.free()
