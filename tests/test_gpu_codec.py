"""GPU parity: dequantisation through the C ABI must be bit-exact against the
oracle (dequant.zig:19-47, 316-390, 632-659)."""
import numpy as np
import pytest

import mmhip as mm

pytestmark = pytest.mark.gpu


def _same_bits(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    na, nb = np.isnan(a), np.isnan(b)
    assert np.array_equal(na, nb), "NaN positions differ"
    bad = np.nonzero(a[~na].view(np.uint32) != b[~na].view(np.uint32))[0]
    assert bad.size == 0, f"{bad.size} values differ, first at {bad[:8]}: {a[~na][bad[:4]]} vs {b[~na][bad[:4]]}"


@pytest.mark.parametrize("rows,cols", [(1536, 2048), (2048, 1536)])
def test_dequant_iq2_xxs_config_bit_exact(ctx, orc, rows, cols):
    rng = np.random.default_rng(100 + rows)
    raw = mm.make_iq2_xxs(rng, rows, cols)
    n = rows * cols
    _same_bits(ctx.dequantize(raw, mm.IQ2_XXS, n), orc.dequantize(raw, orc.IQ2_XXS, n))


def test_dequant_q8_0_config_bit_exact(ctx, orc):
    rng = np.random.default_rng(5)
    raw = mm.make_q8_0(rng, 1536, 2048)
    n = 1536 * 2048
    ref = orc.dequantize(raw, orc.Q8_0, n)
    _same_bits(ctx.dequantize(raw, mm.Q8_0, n), ref)


def test_dequant_q8_0_every_scale_code(ctx, orc):
    """All 65,536 f16 scale codes (subnormals, Inf, NaN included)."""
    codes = np.arange(65536, dtype=np.uint32)
    q = ((np.arange(32) * 37) % 255 - 127).astype(np.int8)
    blocks = np.empty((65536, 34), dtype=np.uint8)
    blocks[:, 0:2] = codes.astype(np.uint16).view(np.uint8).reshape(-1, 2)
    blocks[:, 2:] = np.broadcast_to(q.view(np.uint8), (65536, 32))
    raw = blocks.reshape(-1)
    n = 65536 * 32
    _same_bits(ctx.dequantize(raw, mm.Q8_0, n), orc.dequantize(raw, orc.Q8_0, n))


def test_dequant_iq2_every_scale_code(ctx, orc):
    """Every f16 code as the superblock scale d (random qs)."""
    rng = np.random.default_rng(6)
    blocks = mm.make_iq2_xxs(rng, 256, 65536 // 256 * 256).reshape(65536, 66)
    blocks[:, 0:2] = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.uint8).reshape(-1, 2)
    raw = blocks.reshape(-1)
    _same_bits(ctx.dequantize(raw, mm.IQ2_XXS, 65536 * 256), orc.dequantize(raw, orc.IQ2_XXS, 65536 * 256))


def test_dequant_f16_every_code(ctx, orc):
    raw = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.uint8)
    _same_bits(ctx.dequantize(raw, mm.F16, 65536), orc.dequantize(raw, orc.F16, 65536))


@pytest.mark.parametrize("n", [1, 31, 32, 33, 255, 257, 4096 + 7])
def test_dequant_ragged_lengths(ctx, orc, n):
    """Element counts that end inside a block (dequantize(n) with a partial
    last block, dequant.zig:358-390)."""
    rng = np.random.default_rng(n)
    raw = mm.make_q8_0(rng, 1, ((n + 31) // 32) * 32)
    _same_bits(ctx.dequantize(raw, mm.Q8_0, n), orc.dequantize(raw, orc.Q8_0, n))
    raw2 = mm.make_iq2_xxs(rng, 1, ((n + 255) // 256) * 256)
    _same_bits(ctx.dequantize(raw2, mm.IQ2_XXS, n), orc.dequantize(raw2, orc.IQ2_XXS, n))


def test_dequant_dev_twin_matches_host_path(ctx, orc):
    rng = np.random.default_rng(7)
    raw = mm.make_iq2_xxs(rng, 64, 512)
    n = 64 * 512
    draw = mm.DeviceArray.from_numpy(ctx, raw)
    dout = mm.DeviceArray(ctx, n * 4)
    ctx.dequantize_dev(dout, draw, mm.IQ2_XXS, n)
    ctx.synchronize()
    _same_bits(dout.to_numpy(np.float32, n), orc.dequantize(raw, orc.IQ2_XXS, n))
    draw.free()
    dout.free()


def test_unsupported_type_is_an_error(ctx):
    with pytest.raises(mm.MmhipError) as e:
        ctx.dequantize(np.zeros(144, np.uint8), 12, 256)   # Q4_K: not on this path
    assert e.value.code == mm.ERR_UNSUPPORTED
