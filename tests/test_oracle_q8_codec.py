"""The oracle's Q8_0 quantiser (quantizeQ8_0, dequant.zig:98-130; KVCache.put's
Q8_0 branch, kv_cache.zig:289-349) against facts that do not restate it:
the reference's own round-trip test, the already pinned f32ToF16 for the
stored scale (and exact integer truncation where the reference's subnormal
branch has no defined result), the nearest integer to x / d found by search
with ties away from zero, and the special cases of the format."""
import numpy as np
import pytest


def _blocks(raw):
    b = raw.reshape(-1, 34)
    d = b[:, 0].astype(np.uint16) | (b[:, 1].astype(np.uint16) << 8)
    return d, b[:, 2:].view(np.int8)


def test_kv_cache_quantization_roundtrip_kat(orc):
    """kv_cache.zig:686-719: kv_comp[i] = 0.5 i (kv_lora_rank 512), k_pe[i] =
    0.25 i (rope dim 64); put then get is within 5% + 1e-2 of the input."""
    for n, step in ((512, 0.5), (64, 0.25)):
        x = (step * np.arange(n)).astype(np.float32)
        y = orc.dequantize_q8_0_rows(orc.quantize_q8_0_rows(x, n), 1, n)[0]
        assert np.all(np.abs(y - x) < 0.05 * np.abs(x) + 1e-2)


def _expected_scale_bits(orc, d32):
    """f32ToF16 of d: the pinned converter on the normal range; below 2^-14
    the subnormal result truncated toward zero, from exact float64 arithmetic
    (which also gives the reference's flush to zero below 2^-25)."""
    if d32 >= np.float32(2.0 ** -14):
        h, defect = orc.f32_to_f16(float(d32))
        assert not defect
        return h
    return int(np.floor(float(d32) / 2.0 ** -24))


def _nearest_away(v):
    """Nearest integer to v (float64 of an f32 quotient), ties away from zero."""
    lo, hi = np.floor(v), np.ceil(v)
    dl, dh = v - lo, hi - v
    if dl < dh:
        return lo
    if dh < dl:
        return hi
    return hi if v > 0 else lo


@pytest.mark.parametrize("seed,scale", [(1, 1.0), (2, 1e-3), (3, 300.0), (4, 4e-6)])
def test_quantize_blocks_against_definition(orc, seed, scale):
    rng = np.random.default_rng(seed)
    n = 32 * 40 + 13  # a partial last block
    x = (rng.standard_normal(n) * scale).astype(np.float32)
    x[:32] = 0.0  # an all-zero block
    # Exact ties: the block's maximum is 127 * 2^k, so d = 2^k exactly and
    # every other value sits halfway between two integers times d.
    s2 = np.float32(2.0 ** np.round(np.log2(scale)))
    x[64:96] = (np.arange(32, dtype=np.float32) - np.float32(15.5)) * s2
    x[95] = np.float32(127.0) * s2
    d16, qs = _blocks(orc.quantize_q8_0(x))
    for b in range(d16.size):
        vals = x[32 * b:32 * b + 32]
        max_abs = np.float32(np.max(np.abs(vals))) if vals.size else np.float32(0)
        d = np.float32(max_abs / np.float32(127.0)) if max_abs > 0 else np.float32(0)
        assert d16[b] == _expected_scale_bits(orc, d), b
        for j in range(32):
            if j >= vals.size or d == 0:
                assert qs[b, j] == 0
                continue
            quo = np.float32(vals[j] / d)  # the reference divides by the f32 d
            q = int(np.clip(_nearest_away(float(quo)), -127, 127))
            assert qs[b, j] == q, (b, j, vals[j], d)
        if d > 0:
            assert abs(int(qs[b, np.argmax(np.abs(vals))])) == 127


def test_zero_nan_and_padding(orc):
    x = np.zeros(40, dtype=np.float32)
    x[33] = np.nan
    x[35] = 2.0
    d16, qs = _blocks(orc.quantize_q8_0(x))
    assert d16[0] == 0 and not qs[0].any()  # all-zero block
    h, _ = orc.f32_to_f16(2.0 / 127.0)
    assert d16[1] == h  # the NaN does not take part in the maximum
    assert qs[1, 1] == 0 and qs[1, 3] == 127 and not qs[1, 8:].any()  # NaN -> 0, padding zero


def test_subnormal_scale_truncates(orc):
    """max|x| = 1e-4: d = 7.9e-7 lies in the f16 subnormal range, where the
    reference's converter overflows; the stored scale is the truncated value."""
    x = np.zeros(32, dtype=np.float32)
    x[5] = np.float32(1e-4)
    x[6] = np.float32(-3e-5)
    d16, qs = _blocks(orc.quantize_q8_0(x))
    d = np.float32(np.float32(1e-4) / np.float32(127.0))
    assert d16[0] == int(np.floor(float(d) / 2.0 ** -24))
    assert qs[0, 5] == 127 and qs[0, 6] == int(_nearest_away(float(np.float32(np.float32(-3e-5) / d))))



def test_subnormal_scale_ranges_against_reference_codes(orc):
    """The reference's subnormal branch (dequant.zig:76-77) computes
    m = (mant | 2^23) >> (1 - exp16) and returns (sign << 15) | m via @intCast.
    Worked by hand from those lines:
      d = 2^-20   (exp16 = -5): m = 2^23 >> 6 = 2^17 > 0xFFFF -> @intCast traps;
      d = 2^-22   (exp16 = -7): m = 2^23 >> 8 = 0x8000 -> code 0x8000 (-0.0);
      d = 1.5 * 2^-23 (exp16 = -8): m = 0xC00000 >> 9 = 0x6000 -> 512.0;
      d = 2^-25   (exp16 = -10): m = 2^23 >> 11 = 0x1000 -> 2^-11.
    quantizeQ8_0 here stores the subnormal scale truncated toward zero
    instead (d / 2^-24 rounded down), a deliberate fix: next to each
    reference code, the stored one."""
    cases = [(2.0 ** -20, None, 0x0010), (2.0 ** -22, 0x8000, 0x0004), (1.5 * 2.0 ** -23, 0x6000, 0x0003),
             (2.0 ** -25, 0x1000, 0x0000)]
    for d, ref_code, stored in cases:
        h, defect = orc.f32_to_f16(d)
        if ref_code is None:
            assert defect == 1
        else:
            assert defect == 2 and h == ref_code, (d, hex(h))
        # a block whose max |x| is 127 d: d = max / 127 is exact in f32
        x = np.zeros(32, dtype=np.float32)
        x[3] = np.float32(127.0 * d)
        d16, qs = _blocks(orc.quantize_q8_0(x))
        assert d16[0] == stored == int(np.floor(d / 2.0 ** -24)), (d, hex(int(d16[0])))
        assert qs[0, 3] == 127
