"""Operator planner (OpScheduler / LayerPlan, scheduler.zig:265-552): host logic.

The reference's own tests (scheduler.zig:556-735) are mirrored where this
backend keeps the reference's rules; the GPU rules it adds are tested beside
them. Critical-path values are worked out by hand from the rule at 313-333.
"""
import pytest

import mmhip as mm

pytestmark = []

HP = dict(hidden_size=2048, intermediate_size=1536, num_heads=16, head_dim=128, leading_dense_layers=1,
          n_routed_experts=64)
OP, PREC = mm.OP, mm.PREC
CPU, GPU, NPU = mm.BACKEND_CPU, mm.BACKEND_GPU, mm.BACKEND_NPU


@pytest.fixture(scope="module", autouse=True)
def _lib():
    mm.load_library()


def backends(plan):
    return [(o.op, o.backend) for o in plan]


def test_all_cpu_without_accelerators():
    """'OpScheduler planLayer all CPU when no accel' (scheduler.zig:622-645)."""
    for layer in (0, 1, 5):
        plan = mm.plan_layer(layer, **HP)
        assert plan and all(o.backend == CPU for o in plan)
        assert mm.plan_device_mask(plan) == 0b001


def test_npu_only_keeps_the_reference_rules():
    """Dense layer with an NPU and no GPU: gate/up on the NPU, silu on the CPU,
    down on the CPU (scheduler.zig:436-468); attention stays on the CPU
    (blacklisted, 369-372, 411-419)."""
    plan = mm.plan_layer(0, has_npu=True, **HP)
    assert backends(plan) == [(OP["rmsNorm"], CPU), (OP["attention"], CPU), (OP["rmsNorm"], CPU),
                              (OP["ffn_gate_up"], NPU), (OP["siluMul"], CPU), (OP["ffn_down"], CPU)]
    assert [o.sync_after for o in plan] == [0, 0, 0, 1, 0, 1]


def test_gpu_takes_the_ffn():
    """With a GPU (the HIP backend) gate/up, silu*up and down run on it, dense
    or MoE (shared expert), and no sync sits between them."""
    for layer in (0, 3):
        plan = mm.plan_layer(layer, has_gpu=True, has_npu=True, **HP)
        assert backends(plan)[3:] == [(OP["ffn_gate_up"], GPU), (OP["siluMul"], GPU), (OP["ffn_down"], GPU)]
        assert [o.sync_after for o in plan][3:] == [0, 0, 1]
        assert mm.plan_device_mask(plan) == 0b011
    # 'uses NPU and GPU when available' (648-676): GPU present -> GPU and CPU.
    plan = mm.plan_layer(0, has_gpu=True, has_npu=True, **HP)
    assert any(o.backend == GPU for o in plan)


def test_heavy_throttle_falls_back_to_cpu():
    """'OpScheduler heavy throttle falls back to CPU' (679-703)."""
    for layer in (0, 2):
        plan = mm.plan_layer(layer, has_gpu=True, has_npu=True, throttle_level=3, **HP)
        assert all(o.backend == CPU for o in plan if o.op != OP["attention"])
    # other levels keep the GPU
    for level in (0, 1, 2):
        plan = mm.plan_layer(2, has_gpu=True, throttle_level=level, **HP)
        assert plan[-1].backend == GPU


def test_perf_db_values_are_used():
    """'OpScheduler with perf db uses recorded values' (706-735): rmsNorm at
    dim 2048 recorded at 42 us; GPU ops use the recorded gpu_us."""
    db = [(OP["rmsNorm"], PREC["f32"], (0, 0, 0, 2048), 42, 0),
          (OP["matVecMulQ8_0"], PREC["q8_0"], (1536, 0, 2048, 0), 900, 7),
          (OP["matVecMulQ8_0"], PREC["iq2_xxs"], (2048, 0, 1536, 0), 800, 5)]
    plan = mm.plan_layer(0, perf_db=db, **HP)
    assert [o.estimated_us for o in plan if o.op == OP["rmsNorm"]] == [42, 42]
    assert plan[3].estimated_us == 900  # CPU gate/up -> cpu_us
    plan = mm.plan_layer(0, perf_db=db, has_gpu=True, **HP)
    assert plan[3].estimated_us == 7    # GPU gate/up -> gpu_us
    plan = mm.plan_layer(0, perf_db=db, has_gpu=True, weight_precision=PREC["iq2_xxs"], **HP)
    assert plan[3].precision == PREC["iq2_xxs"] and plan[5].estimated_us == 5


def test_fallback_estimates():
    """fallbackEstimate (523-537): matVecMulQ8_0 = m k / 40000; attention =
    m n k / 2e6; 1-D ops read m and n only and come out 0."""
    plan = mm.plan_layer(0, **HP)
    est = {(o.op, o.shape.m, o.shape.k): o.estimated_us for o in plan}
    assert est[(OP["ffn_gate_up"], 1536, 2048)] == 1536 * 2048 // 40000
    assert est[(OP["ffn_down"], 2048, 1536)] == 2048 * 1536 // 40000
    assert est[(OP["attention"], 16, 128)] == 16 * 128 * 128 // 2000000
    assert est[(OP["rmsNorm"], 0, 0)] == 0 and est[(OP["siluMul"], 0, 0)] == 0
    assert mm.plan_layer(0, seq_len_hint=4096, **HP)[1].shape.k == 4096


def test_critical_path_rule():
    """estimatedCriticalPathUs (313-333) on the reference's own example
    (572-603): rmsNorm cpu 50 | matVec npu 150 (sync) | silu cpu 20 ->
    50 + max(150, 20) = 200; and a same-backend chain adds up."""
    s = mm.op_schedule
    ops = [s(OP["rmsNorm"], CPU, PREC["f32"], 50, False), s(OP["matVecMulQ8_0"], NPU, PREC["q8_0"], 150, True),
           s(OP["siluMul"], CPU, PREC["f32"], 20, False)]
    assert mm.plan_critical_path_us(ops) == 200
    chain = [s(OP["rmsNorm"], CPU, 2, 10, False), s(OP["rmsNorm"], CPU, 2, 15, False), s(OP["dot"], GPU, 2, 7, True),
             s(OP["dot"], GPU, 2, 3, False)]
    assert mm.plan_critical_path_us(chain) == (10 + 15) + (7 + 3)
    assert mm.plan_critical_path_us([]) == 0


def test_device_mask():
    """'LayerPlan deviceMask' (606-619)."""
    s = mm.op_schedule
    ops = [s(OP["rmsNorm"], CPU, 2, 10, False), s(OP["ffn_gate_up"], NPU, 0, 20, False),
           s(OP["ffn_down"], GPU, 0, 30, False)]
    assert mm.plan_device_mask(ops) == 0b111


def test_invalid_arguments():
    with pytest.raises(mm.MmhipError):
        mm.plan_layer(0, weight_precision=PREC["f32"], **HP)
