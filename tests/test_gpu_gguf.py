"""Device-resident weights from a GGUF file (gguf.loadFromFile + Model.bindLayer,
gguf.zig:368-413, model.zig:289-395): a MoE layer bound by tensor name from a
file written by tests/gguf_writer.py gives the same bits, routes and expert
counts as the same layer built from host arrays, and the oracle's moeFFN's
routes and outputs (1e-3 max-abs-rel, as the MoE tests), and a tensor uploaded by name gives the
same GEMV bits as the same bytes uploaded from the host."""
import numpy as np
import pytest

import gguf_writer as gw
import mmhip as mm

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("fmt,shared_fmt", [(mm.IQ2_XXS, mm.Q8_0), (mm.Q8_0, None)])
def test_moe_layer_from_gguf(ctx, orc, tmp_path, fmt, shared_fmt):
    rng = np.random.default_rng(71 + fmt)
    hidden, inter, n_exp, sh_inter, layer = 512, 256, 16, 512, 3
    router = rng.normal(0.0, 0.02, (n_exp, hidden)).astype(np.float32)
    gate = mm.make_weight(rng, fmt, inter, hidden, n_exp)
    up = mm.make_weight(rng, fmt, inter, hidden, n_exp)
    down = mm.make_weight(rng, fmt, hidden, inter, n_exp)
    p = f"blk.{layer}."
    tensors = [(p + "ffn_gate_inp.weight", [hidden, n_exp], mm.F32, router),
               (p + "ffn_gate_exps.weight", [hidden, inter, n_exp], fmt, gate),
               (p + "ffn_up_exps.weight", [hidden, inter, n_exp], fmt, up),
               (p + "ffn_down_exps.weight", [inter, hidden, n_exp], fmt, down)]
    shared = None
    if shared_fmt is not None:
        shared = (mm.make_weight(rng, shared_fmt, sh_inter, hidden), mm.make_weight(rng, shared_fmt, sh_inter, hidden),
                  mm.make_weight(rng, shared_fmt, hidden, sh_inter))
        tensors += [(p + "ffn_gate_shexp.weight", [hidden, sh_inter], shared_fmt, shared[0]),
                    (p + "ffn_up_shexp.weight", [hidden, sh_inter], shared_fmt, shared[1]),
                    (p + "ffn_down_shexp.weight", [sh_inter, hidden], shared_fmt, shared[2])]
    meta = [("general.architecture", gw.STRING, "deepseek2"), ("deepseek2.expert_weights_scale", gw.F32, 1.8)]
    gw.write(tmp_path / "moe.gguf", meta, tensors)
    print(f"gguf moe layer fmt={fmt} shared={shared_fmt}", flush=True)
    with mm.Gguf(tmp_path / "moe.gguf") as g:
        for name, _, _, data in tensors:
            assert np.array_equal(g.tensor_bytes(name), np.ascontiguousarray(data).view(np.uint8).reshape(-1)), name
        from_file = mm.MoeLayer.from_gguf(ctx, g, layer)
    # The mapping is closed: the layer holds device copies only.
    from_host = mm.MoeLayer(ctx, hidden=hidden, inter=inter, n_experts=n_exp, expert_type=fmt, router=router,
                            gate=gate, up=up, down=down, shared=shared,
                            shared_inter=sh_inter if shared else None, shared_type=shared_fmt,
                            routed_scaling_factor=float(np.float32(1.8)))
    try:
        for t in (1, 24):
            h = rng.normal(0.0, 1.0, (t, hidden)).astype(np.float32)
            a = from_file.ffn(h)
            b = from_host.ffn(h)
            c = orc.Moe(hidden=hidden, inter=inter, n_experts=n_exp, expert_type=fmt, router=router, gate=gate,
                        up=up, down=down, shared=shared, shared_inter=sh_inter if shared else None,
                        shared_type=shared_fmt, routed_scaling_factor=float(np.float32(1.8))).ffn(h)
            assert np.array_equal(a[1], c[1])  # no near-ties at these seeds
            assert mm.max_abs_rel(a[0], c[0]) <= 1e-3
            for x, y in zip(a, b):
                assert np.array_equal(x.view(np.uint32), y.view(np.uint32)), t
        assert np.array_equal(from_file.expert_counts(), from_host.expert_counts())
    finally:
        from_file.free()
        from_host.free()


def test_moe_layer_from_gguf_missing_tensor(ctx, tmp_path):
    rng = np.random.default_rng(3)
    gate = mm.make_weight(rng, mm.Q8_0, 64, 256, 4)
    gw.write(tmp_path / "partial.gguf", [], [("blk.0.ffn_gate_exps.weight", [256, 64, 4], mm.Q8_0, gate)])
    with mm.Gguf(tmp_path / "partial.gguf") as g:
        with pytest.raises(mm.MmhipError) as e:
            mm.MoeLayer.from_gguf(ctx, g, 0)
        assert "ffn_gate_inp" in str(e.value)


@pytest.mark.parametrize("fmt", [mm.Q8_0, mm.IQ2_XXS, mm.F32])
def test_upload_tensor_by_name(ctx, tmp_path, fmt):
    rng = np.random.default_rng(90 + fmt)
    rows, cols, count = 576, 2048, 3
    raw = mm.make_weight(rng, fmt, rows, cols, count)
    gw.write(tmp_path / "w.gguf", [("general.alignment", gw.U32, 64)],
             [("output_norm.weight", [5], mm.F32, np.ones(5, np.float32)),
              ("blk.0.attn_kv_a_mqa.weight", [cols, rows, count], fmt, raw)], alignment=64)
    print(f"gguf upload fmt={fmt}", flush=True)
    with mm.Gguf(tmp_path / "w.gguf") as g:
        w_file = ctx.upload_gguf(g, "blk.0.attn_kv_a_mqa.weight")
    w_host = ctx.upload(raw, fmt, rows, cols, count)
    x = mm.DeviceArray.from_numpy(ctx, rng.normal(0.0, 1.0, (count, cols)).astype(np.float32))
    ya, yb = mm.DeviceArray(ctx, count * rows * 4), mm.DeviceArray(ctx, count * rows * 4)
    try:
        assert (w_file.rows, w_file.cols, w_file.count) == (rows, cols, count)
        assert w_file.device_bytes == w_host.device_bytes
        ctx.gemv_batched_dev(w_file, 0, count, x, cols, ya, rows)
        ctx.gemv_batched_dev(w_host, 0, count, x, cols, yb, rows)
        ctx.synchronize()
        a, b = ya.to_numpy(np.float32, count * rows), yb.to_numpy(np.float32, count * rows)
        assert np.isfinite(a).all() and np.array_equal(a.view(np.uint32), b.view(np.uint32))
    finally:
        for o in (x, ya, yb, w_file, w_host):
            o.free()


def test_upload_rejects_partial_block_rows(ctx, tmp_path):
    """Rows of 48 Q8_0 values would share a block: refused before any copy."""
    gw.write(tmp_path / "p.gguf", [], [("w", [48, 2], mm.Q8_0, np.zeros(3 * 34, np.uint8))])
    with mm.Gguf(tmp_path / "p.gguf") as g:
        assert g.tensor("w")["data"]
        with pytest.raises(mm.MmhipError) as e:
            ctx.upload_gguf(g, "w")
        assert "whole number of blocks" in str(e.value)


@pytest.mark.parametrize("fmt", [mm.Q8_0, mm.IQ2_XXS])
def test_upload_stacked_rows(ctx, tmp_path, fmt):
    """attn_q_a [768 x 2048] and attn_kv_a_mqa [576 x 2048] stacked into one
    weight from the file: the same bits as each uploaded and run alone."""
    rng = np.random.default_rng(120 + fmt)
    qa, kva = mm.make_weight(rng, fmt, 768, 2048), mm.make_weight(rng, fmt, 576, 2048)
    names = ["blk.1.attn_q_a.weight", "blk.1.attn_kv_a_mqa.weight"]
    gw.write(tmp_path / "a.gguf", [], [(names[0], [2048, 768], fmt, qa), ("blk.1.attn_norm.weight", [7], mm.F32,
                                                                          np.ones(7, np.float32)),
                                       (names[1], [2048, 576], fmt, kva)])
    print(f"gguf stacked rows fmt={fmt}", flush=True)
    with mm.Gguf(tmp_path / "a.gguf") as g:
        w = ctx.upload_gguf_rows(g, names)
        with pytest.raises(mm.MmhipError):
            ctx.upload_gguf_rows(g, [names[0], "blk.1.attn_norm.weight"])  # another type and row length
    parts = [ctx.upload(qa, fmt, 768, 2048), ctx.upload(kva, fmt, 576, 2048)]
    x = mm.DeviceArray.from_numpy(ctx, rng.standard_normal(2048).astype(np.float32))
    y, y0, y1 = mm.DeviceArray(ctx, 1344 * 4), mm.DeviceArray(ctx, 768 * 4), mm.DeviceArray(ctx, 576 * 4)
    try:
        assert w.rows == 1344 and w.cols == 2048
        ctx.gemv_batched_dev(w, 0, 1, x, 0, y, 0)
        ctx.gemv_batched_dev(parts[0], 0, 1, x, 0, y0, 0)
        ctx.gemv_batched_dev(parts[1], 0, 1, x, 0, y1, 0)
        ctx.synchronize()
        a = y.to_numpy(np.float32, 1344)
        b = np.concatenate([y0.to_numpy(np.float32, 768), y1.to_numpy(np.float32, 576)])
        assert np.isfinite(a).all() and np.array_equal(a.view(np.uint32), b.view(np.uint32))
    finally:
        for o in [x, y, y0, y1, w] + parts:
            o.free()
