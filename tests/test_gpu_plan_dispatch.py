"""A layer plan executed through the HIP backend: OpScheduler.planLayer
(scheduler.zig:473-501, with this backend's GPU rule) sends a MoE layer's
ffn_gate_up, siluMul and ffn_down to the GPU, and PlanDispatch (the body of
HeteroExecutor.dispatchGpu, hetero_executor.zig:154-159, as
zig/hip_backend.zig's PlanDispatch) runs them on a device-resident MoeLayer.
The executor loop below plays executeLayer (hetero_executor.zig:88-127): GPU
ops go to PlanDispatch, the rest (RMSNorm, attention) stay with the engine's
CPU path and are not part of this check. After ffn_down the hidden state
must equal the oracle's moeFFN of the same input."""
import numpy as np
import pytest

import mmhip as mm

pytestmark = pytest.mark.gpu

H, I, E = 512, 256, 16
HP = dict(hidden_size=H, intermediate_size=I, num_heads=4, head_dim=64, leading_dense_layers=1,
          n_routed_experts=E, weight_precision=mm.PREC["iq2_xxs"])


@pytest.fixture(scope="module")
def layer(ctx, orc):
    rng = np.random.default_rng(4242)
    kw = dict(hidden=H, inter=I, n_experts=E, expert_type=mm.IQ2_XXS,
              router=rng.normal(0.0, 0.05, (E, H)).astype(np.float32),
              gate=mm.make_iq2_xxs(rng, I, H, E), up=mm.make_iq2_xxs(rng, I, H, E),
              down=mm.make_iq2_xxs(rng, H, I, E),
              shared=(mm.make_iq2_xxs(rng, I, H), mm.make_iq2_xxs(rng, I, H), mm.make_iq2_xxs(rng, H, I)),
              shared_inter=I)
    gpu = mm.MoeLayer(ctx, **kw)
    cpu = orc.Moe(**kw)
    yield gpu, cpu
    gpu.free()


def execute(plan, dispatch, hidden):
    """executeLayer's loop over the plan: GPU ops through the dispatch."""
    ran = []
    for op in plan:
        if op.backend == mm.BACKEND_GPU:
            dispatch.dispatch_gpu(op, hidden)
            ran.append(op.op)
    return ran


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_gpu_ops_of_a_moe_layer_plan(layer, seed):
    gpu, cpu = layer
    plan = mm.plan_layer(3, has_gpu=True, **HP)
    rng = np.random.default_rng(100 + seed)
    x = rng.standard_normal(H).astype(np.float32)
    hidden = x.copy()
    d = mm.PlanDispatch(gpu)
    try:
        ran = execute(plan, d, hidden)
    finally:
        d.release()
    assert ran == [mm.OP["ffn_gate_up"], mm.OP["siluMul"], mm.OP["ffn_down"]]
    ref = cpu.ffn(x[None, :])[0].reshape(-1)
    assert mm.max_abs_rel(hidden, ref) <= 1e-3


def test_a_layer_runs_through_one_path(layer):
    """The reference plans only the shared expert for a MoE layer and leaves
    the routed experts to moeFFN (scheduler.zig:466-501); here the plan's FFN
    ops run the whole layer, so a layer bound to a PlanDispatch refuses
    moeFFN's direct call (and a second binding) until it is released, and no
    token's routed experts run twice."""
    gpu, cpu = layer
    rng = np.random.default_rng(7)
    x = rng.standard_normal(H).astype(np.float32)
    d = mm.PlanDispatch(gpu)
    try:
        with pytest.raises(mm.MmhipError) as e:
            gpu.ffn(x[None, :])
        assert e.value.code == mm.ERR_INVALID
        with pytest.raises(mm.MmhipError) as e:
            mm.PlanDispatch(gpu)
        assert e.value.code == mm.ERR_INVALID
        hidden = x.copy()
        execute(mm.plan_layer(3, has_gpu=True, **HP), d, hidden)
    finally:
        d.release()
    direct = gpu.ffn(x[None, :])[0].reshape(-1)
    np.testing.assert_array_equal(direct.view(np.uint32), hidden.view(np.uint32))
    assert mm.max_abs_rel(direct, cpu.ffn(x[None, :])[0].reshape(-1)) <= 1e-3


def test_dispatch_errors(layer):
    gpu, _ = layer
    d = mm.PlanDispatch(gpu)
    h = np.zeros(H, np.float32)
    try:
        for name, code in (("siluMul", mm.ERR_INVALID), ("ffn_down", mm.ERR_INVALID),
                           ("attention", mm.ERR_UNSUPPORTED), ("rmsNorm", mm.ERR_UNSUPPORTED)):
            with pytest.raises(mm.MmhipError) as e:
                d.dispatch_gpu(mm.op_schedule(mm.OP[name], mm.BACKEND_GPU, 0, 0, False), h)
            assert e.value.code == code
    finally:
        d.release()
    # A dense layer (no MoeLayer) keeps its FFN on the CPU path.
    with pytest.raises(mm.MmhipError) as e:
        mm.PlanDispatch(None).dispatch_gpu(mm.op_schedule(mm.OP["ffn_gate_up"], mm.BACKEND_GPU, 0, 0, False), h)
    assert e.value.code == mm.ERR_UNSUPPORTED
