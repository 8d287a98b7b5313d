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


@pytest.mark.parametrize("fmt,raw_off,out_off", [(mm.Q8_0, 1, 4), (mm.Q8_0, 2, 0), (mm.IQ2_XXS, 1, 4),
                                                  (mm.IQ2_XXS, 0, 8)])
def test_dequant_dev_misaligned_pointers(ctx, orc, fmt, raw_off, out_off):
    """mmhip_dequantize_dev with raw blocks at odd / 2-byte offsets and an
    output that is not 16-byte aligned (the scalar-store and 2-byte-load
    paths), against the oracle bit for bit."""
    rng = np.random.default_rng(raw_off * 10 + out_off)
    n = 3 * 256 + 64
    raw = mm.make_weight(rng, fmt, 1, ((n + 255) // 256) * 256)
    buf = np.zeros(raw.size + 16, np.uint8)
    buf[raw_off:raw_off + raw.size] = raw
    draw = mm.DeviceArray.from_numpy(ctx, buf)
    dout = mm.DeviceArray(ctx, n * 4 + 64)
    try:
        mm.check(ctx.lib.mmhip_dequantize_dev(ctx.handle, dout.ptr + out_off, draw.ptr + raw_off, fmt, n),
                 "mmhip_dequantize_dev")
        ctx.synchronize()
        got = dout.to_numpy(np.uint8, n * 4 + out_off)[out_off:].view(np.float32)
        _same_bits(got, orc.dequantize(raw, fmt, n))
    finally:
        draw.free()
        dout.free()


def test_unsupported_type_is_an_error(ctx):
    with pytest.raises(mm.MmhipError) as e:
        ctx.dequantize(np.zeros(144, np.uint8), 12, 256)   # Q4_K: not on this path
    assert e.value.code == mm.ERR_UNSUPPORTED


# ---- Q8_0 quantiser (quantizeQ8_0, dequant.zig:98-130; KVCache.put /
# getKVCompressed's Q8_0 branches, kv_cache.zig:225-349): bit-exact ----

def _q8_rows_input(rng, n_rows, row_len, scale):
    """Random rows with the cases the format has: an all-zero block, exact
    ties (a block whose maximum is 127 * 2^k, other values half-integers of
    2^k), a NaN and, with small scales, block scales in the f16 subnormal
    range."""
    x = (rng.standard_normal((n_rows, row_len)) * scale).astype(np.float32)
    if row_len >= 64:
        x[0, :32] = 0.0
        s2 = np.float32(2.0 ** np.round(np.log2(scale)))
        x[0, 32:64] = (np.arange(32, dtype=np.float32) - np.float32(15.5)) * s2
        x[0, 63] = np.float32(127.0) * s2
    if n_rows > 1:
        x[1, row_len // 2] = np.nan
    return x


@pytest.mark.parametrize("n_rows,row_len,scale", [(1, 512, 1.0), (7, 64, 0.25), (33, 100, 3.0), (5, 33, 1e-3),
                                                  (64, 512, 4e-6), (3, 1, 1.0), (257, 576, 30.0)])
def test_q8_0_rows_match_oracle(ctx, orc, n_rows, row_len, scale):
    rng = np.random.default_rng(n_rows * 1000 + row_len)
    x = _q8_rows_input(rng, n_rows, row_len, scale)
    ref = orc.quantize_q8_0_rows(x, row_len)
    # Device twin with a row stride larger than the row.
    stride = row_len + 3
    xs = np.zeros((n_rows, stride), dtype=np.float32)
    xs[:, :row_len] = x
    dx = mm.DeviceArray.from_numpy(ctx, xs)
    db = mm.DeviceArray(ctx, max(ref.size, 4))
    dy = mm.DeviceArray(ctx, n_rows * stride * 4)
    try:
        ctx.quantize_q8_0_rows_dev(db, dx, stride, n_rows, row_len)
        got = db.to_numpy(np.uint8, ref.size)
        np.testing.assert_array_equal(got, ref)
        # And back: getKVCompressed's dequantisation, bit-exact (NaN aside).
        ctx.dequantize_q8_0_rows_dev(dy, stride, db, n_rows, row_len)
        y = dy.to_numpy(np.float32, n_rows * stride).reshape(n_rows, stride)[:, :row_len]
        yr = orc.dequantize_q8_0_rows(ref, n_rows, row_len)
        np.testing.assert_array_equal(y.view(np.uint32), yr.view(np.uint32))
    finally:
        dx.free(); db.free(); dy.free()
    # Host twin over the flattened array (quantizeQ8_0 itself).
    np.testing.assert_array_equal(ctx.quantize_q8_0(x.reshape(-1)), orc.quantize_q8_0(x.reshape(-1)))


def test_q8_0_kv_roundtrip_kat(ctx):
    """kv_cache.zig:686-719 on the device: kv_comp[i] = 0.5 i (512 values),
    k_pe[i] = 0.25 i (64 values); put then get within 5% + 1e-2."""
    for n, step in ((512, 0.5), (64, 0.25)):
        x = (step * np.arange(n)).astype(np.float32)
        dx = mm.DeviceArray.from_numpy(ctx, x)
        db = mm.DeviceArray(ctx, (n // 32) * 34 + 4)
        dy = mm.DeviceArray(ctx, n * 4)
        try:
            ctx.quantize_q8_0_rows_dev(db, dx, n, 1, n)
            ctx.dequantize_q8_0_rows_dev(dy, n, db, 1, n)
            y = dy.to_numpy(np.float32, n)
            assert np.all(np.abs(y - x) < 0.05 * np.abs(x) + 1e-2)
        finally:
            dx.free(); db.free(); dy.free()


def test_q8_0_requantise_is_identity_at_scale(ctx):
    """A KV prefill's worth of rows (16384 positions x 576 values: kv_lora 512
    + rope 64): quantise, dequantise, quantise again gives the same bytes
    (each block's largest |q| is 127, so d * 127 / 127 = d exactly), and the
    round trip stays within half a step of the stored scale."""
    n_rows, row_len = 16384, 576
    rng = np.random.default_rng(77)
    x = rng.standard_normal((n_rows, row_len)).astype(np.float32)
    nbytes = n_rows * (row_len // 32) * 34
    dx = mm.DeviceArray.from_numpy(ctx, x)
    db = mm.DeviceArray(ctx, nbytes)
    db2 = mm.DeviceArray(ctx, nbytes)
    dy = mm.DeviceArray(ctx, x.nbytes)
    try:
        ctx.quantize_q8_0_rows_dev(db, dx, row_len, n_rows, row_len)
        ctx.dequantize_q8_0_rows_dev(dy, row_len, db, n_rows, row_len)
        ctx.quantize_q8_0_rows_dev(db2, dy, row_len, n_rows, row_len)
        b1 = db.to_numpy(np.uint8, nbytes)
        np.testing.assert_array_equal(db2.to_numpy(np.uint8, nbytes), b1)
        y = dy.to_numpy(np.float32, n_rows * row_len).reshape(n_rows, row_len)
        d = (b1.reshape(-1, 34)[:, :2].copy().view(np.float16).astype(np.float32)).reshape(n_rows, row_len // 32)
        step = np.repeat(d, 32, axis=1)
        # |x - d16 q| <= d32 / 2 + 127 |d32 - d16|; d16 is within 2^-11 of d32
        assert np.all(np.abs(x - y) <= step * (0.5 + 127 * 2.0 ** -10) + 1e-30)
    finally:
        dx.free(); db.free(); db2.free(); dy.free()


@pytest.mark.parametrize("n_rows,row_len", [(9, 100), (130, 512)])
def test_q8_0_rows_dequantize_from_2_byte_aligned_blocks(ctx, orc, n_rows, row_len):
    """Blocks are 34 bytes, so a slice of a block array may start 2 bytes past
    a 4-byte boundary; the dequantiser must read it the same way."""
    rng = np.random.default_rng(n_rows + row_len)
    x = rng.standard_normal((n_rows, row_len)).astype(np.float32)
    ref = orc.quantize_q8_0_rows(x, row_len)
    buf = np.zeros(ref.size + 2, dtype=np.uint8)
    buf[2:] = ref
    db = mm.DeviceArray.from_numpy(ctx, buf)
    dy = mm.DeviceArray(ctx, x.nbytes)
    try:
        ctx.dequantize_q8_0_rows_dev(dy, row_len, db, n_rows, row_len, blocks_offset=2)
        y = dy.to_numpy(np.float32, x.size).reshape(n_rows, row_len)
        np.testing.assert_array_equal(y.view(np.uint32), orc.dequantize_q8_0_rows(ref, n_rows, row_len).view(np.uint32))
    finally:
        db.free(); dy.free()


def _near_tie_rows(max_abs):
    """Rows whose quotients x / d sit 0..4 ulp either side of half-integers
    (h * d nudged by whole ulps), with one value per block equal to max_abs so
    that d = max_abs / 127: the cases where an estimated quotient could round
    to a different integer than the correctly rounded one."""
    d = np.float32(np.float32(max_abs) / np.float32(127.0))
    halves = (np.arange(0, 127, dtype=np.float32) + np.float32(0.5))
    vals = []
    for h in halves:
        base = np.float32(h * d)
        for steps in range(-4, 5):
            v = base
            for _ in range(abs(steps)):
                v = np.nextafter(v, np.float32(np.inf if steps > 0 else -np.inf), dtype=np.float32)
            vals.append(v)
            vals.append(-v)
    vals = np.array(vals, dtype=np.float32)
    n_blk = (vals.size + 30) // 31
    rows = np.zeros((n_blk, 32), dtype=np.float32)
    rows.reshape(-1)[:vals.size] = vals
    rows[:, 31] = np.float32(max_abs)
    return rows


@pytest.mark.parametrize("max_abs", [127.0, 100.0, 3.0e-3, 7.25, 1.0e5])
def test_q8_0_near_ties_match_oracle(ctx, orc, max_abs):
    x = _near_tie_rows(max_abs)
    n_rows, row_len = x.shape
    ref = orc.quantize_q8_0_rows(x, row_len)
    dx = mm.DeviceArray.from_numpy(ctx, x)
    db = mm.DeviceArray(ctx, ref.size + 4)
    try:
        ctx.quantize_q8_0_rows_dev(db, dx, row_len, n_rows, row_len)
        np.testing.assert_array_equal(db.to_numpy(np.uint8, ref.size), ref)
    finally:
        dx.free(); db.free()


@pytest.mark.parametrize("max_abs", [1.0e-37, 1.0e-39, 1.0e-41, 1.0e-43, 3.0e-45])
def test_q8_0_subnormal_scales_match_oracle(ctx, orc, max_abs):
    """Blocks whose scale d = max|x| / 127 is an f32 subnormal, with values
    next to half-integer quotients: d loses precision there, so quotients can
    pass 127.5 (clamped) and the fast quotient's bounds are exercised."""
    x = _near_tie_rows(max_abs)
    rng = np.random.default_rng(17)
    x[::3, :31] = (rng.uniform(-1.0, 1.0, (x[::3].shape[0], 31)) * np.float32(max_abs)).astype(np.float32)
    n_rows, row_len = x.shape
    ref = orc.quantize_q8_0_rows(x, row_len)
    dx = mm.DeviceArray.from_numpy(ctx, x)
    db = mm.DeviceArray(ctx, ref.size + 4)
    try:
        ctx.quantize_q8_0_rows_dev(db, dx, row_len, n_rows, row_len)
        np.testing.assert_array_equal(db.to_numpy(np.uint8, ref.size), ref)
    finally:
        dx.free(); db.free()


@pytest.mark.parametrize("scale", [1.0, 1e-4, 50.0])
def test_q8_0_large_random_match_oracle(ctx, orc, scale):
    n_rows, row_len = 7000, 576
    rng = np.random.default_rng(int(scale * 1000) + 9)
    x = (rng.standard_normal((n_rows, row_len)) * scale).astype(np.float32)
    ref = orc.quantize_q8_0_rows(x, row_len)
    dx = mm.DeviceArray.from_numpy(ctx, x)
    db = mm.DeviceArray(ctx, ref.size)
    try:
        ctx.quantize_q8_0_rows_dev(db, dx, row_len, n_rows, row_len)
        got = db.to_numpy(np.uint8, ref.size)
        bad = np.nonzero(got != ref)[0]
        assert bad.size == 0, f"{bad.size} bytes differ, first at {bad[:6]}"
    finally:
        dx.free(); db.free()


def test_q8_0_one_row_past_2_pow_29(ctx, orc):
    """quantize_q8_0 and dequantize over one row of 2^29 + 32,000 values, so
    the row holds 2^24 + 1,000 blocks: the row split must not use 24-bit
    multiplies there (block 2^24 + 999 stays in row 0). Bit-exact against the
    oracle, including the blocks past 2^24."""
    n = (1 << 29) + 32000
    rng = np.random.default_rng(29)
    x = rng.standard_normal(n, dtype=np.float32)
    blocks = ctx.quantize_q8_0(x)
    ref = orc.quantize_q8_0(x)
    bad = np.nonzero(blocks != ref)[0]
    assert bad.size == 0, f"{bad.size} bytes differ, first at {bad[:6]}"
    del x, ref
    got = ctx.dequantize(blocks, mm.Q8_0, n)
    want = orc.dequantize(blocks, orc.Q8_0, n)
    bad = np.nonzero(got.view(np.uint32) != want.view(np.uint32))[0]
    assert bad.size == 0, f"{bad.size} values differ, first at {bad[:6]}"
