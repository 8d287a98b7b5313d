"""Pins the oracle's CPU kernels, routing and MoE FFN: the reference's own
known-answer tests (qmm.zig, math.zig, thermal.zig), float64 recomputation
at the configuration shapes, brute force for top-k and closed forms for the
routing softmax."""
import numpy as np
import pytest

import mmhip as mm


def _q8_blocks(n_blocks, d_bits, qs):
    b = np.zeros((n_blocks, 34), dtype=np.uint8)
    b[:, 0:2] = np.array([d_bits], np.uint16).view(np.uint8)
    b[:, 2:] = np.asarray(qs, dtype=np.int8).reshape(n_blocks, 32).view(np.uint8)
    return b.reshape(-1)


# ---- qmm.zig KATs ----

def test_matmul_q8_0_batch_matches_f32_reference(orc):
    # qmm.zig:142-173
    m, n, k = 4, 8, 64
    d, _ = orc.f32_to_f16(1.0 / 127.0)
    blocks = _q8_blocks(m * 2, d, np.full(m * 2 * 32, 127))
    out = orc.matmul_q8_0(blocks, np.ones((n, k), np.float32), m, n, k)
    assert np.all(np.abs(out - 64.0) <= 0.1)


def test_matmul_q8_0_vs_repeated_matvec(orc):
    # qmm.zig:175-211
    m, n, k = 3, 5, 64
    d, _ = orc.f32_to_f16(0.5 / 127.0)
    qs = np.array([(i * 32 + j) % 127 for i in range(m * 2) for j in range(32)])
    blocks = _q8_blocks(m * 2, d, qs)
    b = (np.arange(n * k) % 7).astype(np.float32) * np.float32(0.3)
    out = orc.matmul_q8_0(blocks, b.reshape(n, k), m, n, k)
    for ni in range(n):
        exp = orc.matvec_q8_0(blocks, b[ni * k:(ni + 1) * k], m, k)
        assert np.all(np.abs(exp - out[:, ni]) <= 0.01)


def test_matvec_q8_0_matches_f32_reference(orc):
    # qmm.zig:213-238
    d, _ = orc.f32_to_f16(1.0 / 127.0)
    blocks = _q8_blocks(8, d, np.full(8 * 32, 127))
    out = orc.matvec_q8_0(blocks, np.ones(64, np.float32), 4, 64)
    assert np.all(np.abs(out - 64.0) <= 0.1)


# ---- float64 recomputation at configuration shapes ----

def _f64_ref(w_f32, x):
    return w_f32.astype(np.float64) @ np.asarray(x, dtype=np.float64)


@pytest.mark.parametrize("rows,cols", [(1536, 2048), (2048, 1536), (37, 96)])
def test_matvec_q8_0_against_float64(orc, rows, cols):
    rng = np.random.default_rng(rows + cols)
    raw = mm.make_q8_0(rng, rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    w = orc.dequantize(raw, orc.Q8_0, rows * ((cols + 31) // 32) * 32).reshape(rows, -1)[:, :cols]
    got = orc.matvec_q8_0(raw, x, rows, cols)
    assert mm.max_abs_rel(got, _f64_ref(w, x)) < 1e-5


def test_matmul_q8_0_against_float64(orc):
    rng = np.random.default_rng(11)
    m, n, k = 96, 64, 2048
    raw = mm.make_q8_0(rng, m, k)
    b = rng.standard_normal((n, k)).astype(np.float32)
    w = orc.dequantize(raw, orc.Q8_0, m * k).reshape(m, k)
    got = orc.matmul_q8_0(raw, b, m, n, k)
    assert mm.max_abs_rel(got, w.astype(np.float64) @ b.astype(np.float64).T) < 1e-5


def test_matmul_q8_0_ragged_k(orc):
    rng = np.random.default_rng(12)
    m, n, k = 5, 7, 70            # tail columns inside the last block
    raw = mm.make_q8_0(rng, m, k)
    b = rng.standard_normal((n, k)).astype(np.float32)
    w = orc.dequantize(raw, orc.Q8_0, m * 96).reshape(m, 96)[:, :k]
    got = orc.matmul_q8_0(raw, b, m, n, k)
    assert mm.max_abs_rel(got, w.astype(np.float64) @ b.astype(np.float64).T) < 1e-5


@pytest.mark.parametrize("rows,cols", [(64, 2048), (5, 7)])
def test_matvec_f32_against_float64(orc, rows, cols):
    rng = np.random.default_rng(3)
    w = rng.standard_normal((rows, cols)).astype(np.float32)
    x = rng.standard_normal(cols).astype(np.float32)
    assert mm.max_abs_rel(orc.matvec_f32(w, x, rows, cols), _f64_ref(w, x)) < 1e-5


def test_unified_seam_iq2_is_dequant_then_f32(orc):
    rng = np.random.default_rng(4)
    raw = mm.make_iq2_xxs(rng, 64, 512)
    x = rng.standard_normal(512).astype(np.float32)
    w = orc.dequantize(raw, orc.IQ2_XXS, 64 * 512).reshape(64, 512)
    got = orc.mat_vec_mul_unified(raw, orc.IQ2_XXS, x, 64, 512)
    assert np.array_equal(got, orc.matvec_f32(w, x, 64, 512))
    assert mm.max_abs_rel(got, _f64_ref(w, x)) < 1e-5


def test_batch_seam_q8_0_is_transposed_matmul(orc):
    rng = np.random.default_rng(5)
    raw = mm.make_q8_0(rng, 48, 128)
    xin = rng.standard_normal((6, 128)).astype(np.float32)
    got = orc.batch_mat_mul_unified(raw, orc.Q8_0, xin, 48, 6, 128)
    assert np.array_equal(got, orc.matmul_q8_0(raw, xin, 48, 6, 128).T)


# ---- math.zig KATs ----

def test_dot_kat(orc):
    assert abs(orc.dot([1.0, 2.0, 3.0], [4.0, 5.0, 6.0]) - 32.0) <= 1e-4   # math.zig:284-287


def test_silu_kat_and_closed_form(orc):
    assert abs(orc.silu(0.0)) <= 1e-4                  # math.zig:256-259
    assert abs(orc.silu(-100.0)) <= 1e-2
    for x in np.linspace(-20, 20, 81):
        assert abs(orc.silu(float(x)) - x / (1 + np.exp(-x))) <= 1e-6 * max(1.0, abs(x))


def test_topk_kat(orc):
    idx, sc = orc.topk([1.0, 5.0, 3.0, 10.0, 2.0, 8.0, 4.0, 7.0], 3)   # math.zig:274-282
    assert list(idx) == [3, 5, 7]
    assert list(sc) == [10.0, 8.0, 7.0]


def test_topk_brute_force(orc):
    rng = np.random.default_rng(9)
    for trial in range(300):
        n = int(rng.integers(1, 65))
        k = int(rng.integers(1, min(n, 4) + 1))
        s = rng.standard_normal(n).astype(np.float32)
        idx, sc = orc.topk(s, k)
        order = np.argsort(-s.astype(np.float64), kind="stable")[:k]
        assert list(idx) == list(order)
        assert np.array_equal(sc, s[order])


def test_topk_ties_follow_the_heap(orc):
    """Tie behaviour of the reference heap (worked by hand from math.zig:142-171):
    [5, 5, 9] with k = 2 evicts the root (index 0) when 9 arrives."""
    idx, _ = orc.topk([5.0, 5.0, 9.0], 2)
    assert sorted(idx.tolist()) == [1, 2]


# ---- routing: Scheduler.route + ThrottleState ----

def test_throttle_table(orc):
    # thermal.zig:157-166 plus the level table (44-72)
    for level, limit, hot_cpu in [(0, 4, 0), (1, 3, 0), (2, 2, 1), (3, 1, 1)]:
        th = orc.throttle(level)
        assert (th.active_expert_limit, th.hot_experts_on_cpu) == (limit, hot_cpu)


@pytest.mark.parametrize("level,scale", [(0, 1.0), (1, 0.83), (2, 0.67), (3, 0.5)])
def test_route_softmax_closed_form(orc, level, scale):
    rng = np.random.default_rng(level)
    s = rng.standard_normal(64).astype(np.float32)
    ids, w, targets, deferred = orc.route(s, level=level, rsf=1.25)
    k = [4, 3, 2, 1][level]
    order = np.argsort(-s.astype(np.float64))[:k]
    assert list(ids) == list(order)
    e = np.exp(s[order].astype(np.float64) - s[order].max())
    ref = e / e.sum() * 1.25 * scale
    assert np.allclose(w, ref, rtol=1e-6, atol=0)
    assert not deferred


def test_route_heavy_with_wider_limit_defers(orc):
    """level heavy with active_expert_limit 4 (fields set independently):
    keep the top-1 expert, renormalise it to the scaling factor, defer."""
    s = np.random.default_rng(1).standard_normal(64).astype(np.float32)
    ids, w, targets, deferred = orc.route(s, level=orc.HEAVY, rsf=1.0, active_expert_limit=4)
    assert deferred
    assert list(targets[1:]) == [orc.TARGET_SKIPPED] * 3
    assert abs(w[0] - 0.5) <= 1e-6


def test_route_stats_and_hot_targets(orc):
    st = orc.Stats(1, 64)
    s = np.zeros(64, np.float32)
    s[[3, 9, 1, 7]] = [4.0, 3.0, 2.0, 1.0]
    ids, w, targets, _ = orc.route(s, stats=st)
    # first token: threshold 0, every expert is hot -> gpu
    assert list(targets) == [orc.TARGET_GPU] * 4
    assert st.s.total_tokens == 1 and st.counts[[3, 9, 1, 7]].tolist() == [1, 1, 1, 1]


# ---- MoE FFN against a float64 recomputation ----

def _moe_case(rng, hidden, inter, n_exp, t, with_shared=True):
    router = (rng.standard_normal((n_exp, hidden)) * 0.02).astype(np.float32)
    gate = mm.make_iq2_xxs(rng, inter, hidden, n_exp)
    up = mm.make_iq2_xxs(rng, inter, hidden, n_exp)
    down = mm.make_iq2_xxs(rng, hidden, inter, n_exp)
    shared = None
    if with_shared:
        shared = (mm.make_iq2_xxs(rng, inter, hidden), mm.make_iq2_xxs(rng, inter, hidden),
                  mm.make_iq2_xxs(rng, hidden, inter))
    h = rng.standard_normal((t, hidden)).astype(np.float32)
    return router, gate, up, down, shared, h


def _moe_f64(orc, hidden, inter, n_exp, router, gate, up, down, shared, h, ids, w):
    def deq(raw, rows, cols, count):
        return orc.dequantize(raw, orc.IQ2_XXS, rows * cols * count).reshape(count, rows, cols).astype(np.float64)
    G, U, D = deq(gate, inter, hidden, n_exp), deq(up, inter, hidden, n_exp), deq(down, hidden, inter, n_exp)
    out = np.zeros((h.shape[0], hidden))
    for t in range(h.shape[0]):
        x = h[t].astype(np.float64)
        for e, wt in zip(ids[t], w[t]):
            g = G[e] @ x
            out[t] += wt * (D[e] @ (g / (1 + np.exp(-g)) * (U[e] @ x)))
        if shared:
            sg, su, sd = deq(shared[0], inter, hidden, 1)[0], deq(shared[1], inter, hidden, 1)[0], deq(shared[2], hidden, inter, 1)[0]
            g = sg @ x
            out[t] += sd @ (g / (1 + np.exp(-g)) * (su @ x))
    return out


def test_moe_ffn_against_float64(orc):
    rng = np.random.default_rng(21)
    hidden, inter, n_exp, t = 512, 256, 16, 3
    router, gate, up, down, shared, h = _moe_case(rng, hidden, inter, n_exp, t)
    moe = orc.Moe(hidden=hidden, inter=inter, n_experts=n_exp, expert_type=orc.IQ2_XXS, router=router,
                  gate=gate, up=up, down=down, shared=shared)
    out, ids, w = moe.ffn(h)
    logits = h.astype(np.float64) @ router.astype(np.float64).T
    for ti in range(t):
        assert list(ids[ti]) == list(np.argsort(-logits[ti])[:4])
    ref = _moe_f64(orc, hidden, inter, n_exp, router, gate, up, down, shared, h, ids, w)
    assert mm.max_abs_rel(out, ref) < 1e-5


def test_moe_ffn_pool_matches_serial(orc):
    rng = np.random.default_rng(22)
    hidden, inter, n_exp, t = 256, 256, 8, 2
    router, gate, up, down, shared, h = _moe_case(rng, hidden, inter, n_exp, t)
    moe = orc.Moe(hidden=hidden, inter=inter, n_experts=n_exp, expert_type=orc.IQ2_XXS, router=router,
                  gate=gate, up=up, down=down, shared=shared)
    pool = orc.Pool(4)
    try:
        a, ia, wa = moe.ffn(h, pool=pool)
    finally:
        pool.close()
    b, ib, wb = moe.ffn(h)
    assert np.array_equal(a, b) and np.array_equal(ia, ib) and np.array_equal(wa, wb)


# ---- sampleGreedy (inference.zig:376-386) ----

def test_sample_greedy_cases(orc):
    f = np.float32
    assert orc.sample_greedy(np.array([1, 3, 3, 2], f)) == 1          # ties keep the earlier index
    assert orc.sample_greedy(np.array([-0.0, 0.0], f)) == 0           # -0 == +0: no takeover
    assert orc.sample_greedy(np.array([0.0, -0.0], f)) == 0
    assert orc.sample_greedy(np.array([np.nan, 5, 9], f)) == 0        # a NaN logits[0] stays
    assert orc.sample_greedy(np.array([1, np.nan, 0.5, 2, np.nan], f)) == 3  # NaN never takes over
    assert orc.sample_greedy(np.array([-np.inf, np.nan, -np.inf], f)) == 0
    assert orc.sample_greedy(np.full(7, 2.5, f)) == 0
    assert orc.sample_greedy(np.array([4.0], f)) == 0


def test_sample_greedy_matches_numpy_first_argmax(orc):
    rng = np.random.default_rng(11)
    for n in (2, 17, 1000, 154880):
        x = rng.integers(-50, 50, n).astype(np.float32)  # many ties
        assert orc.sample_greedy(x) == int(np.argmax(x))
