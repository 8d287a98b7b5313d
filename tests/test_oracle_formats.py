"""Pins the oracle's format functions (dequant.zig / gguf.zig restatement)
against the reference's own known-answer tests and against what IEEE-754 and
the IQ2_XXS format definition fix independently of the oracle's code."""
import os
import re

import numpy as np
import pytest

from conftest import REFERENCE_SRC


# ---- f16ToF32: reference KATs (dequant.zig:663-707) ----

def test_f16_to_f32_subnormal_kats(orc):
    # dequant.zig:663-675
    assert abs(orc.f16_to_f32(0x0001) - 5.9604645e-8) <= 1e-14
    assert abs(orc.f16_to_f32(0x03FF) - 6.097555e-5) <= 1e-8
    assert abs(orc.f16_to_f32(0x0080) - 7.6293945e-6) <= 1e-12


def test_f16_to_f32_comprehensive_kats(orc):
    # dequant.zig:677-707
    assert orc.f16_to_f32(0x0000) == 0.0 and np.signbit(np.float32(orc.f16_to_f32(0x0000))) == False
    assert orc.f16_to_f32(0x8000) == 0.0 and np.signbit(np.float32(orc.f16_to_f32(0x8000)))
    for h, v in [(0x3C00, 1.0), (0x4000, 2.0), (0x3800, 0.5), (0xBC00, -1.0)]:
        assert abs(orc.f16_to_f32(h) - v) <= 1e-4
    assert 0.0 < orc.f16_to_f32(0x03FF) < 0.001
    assert np.isinf(orc.f16_to_f32(0x7C00)) and np.isinf(orc.f16_to_f32(0xFC00))
    assert np.isnan(orc.f16_to_f32(0x7C01))


def test_f16_to_f32_exhaustive_ieee(orc):
    """All 65,536 codes against IEEE binary16 -> binary32 (numpy's exact
    conversion). NaNs are compared by NaN-ness: the reference keeps the
    payload without setting the quiet bit (dequant.zig:41)."""
    codes = np.arange(65536, dtype=np.uint32)
    ref = codes.astype(np.uint16).view(np.float16).astype(np.float32)
    got = np.array([orc.f16_to_f32(int(c)) for c in codes], dtype=np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    # payload preservation of the reference: 0x7C01 -> 0x7F802000 (read through
    # an f32 buffer: a ctypes float return would be widened and quieted)
    out = orc.dequantize(np.array([0x7C01, 0xFE00], np.uint16).view(np.uint8), orc.F16, 2)
    assert out.view(np.uint32).tolist() == [0x7F802000, 0xFFC00000]


def test_f32_to_f16_normal_range_rne(orc):
    # reference test inputs (qmm.zig:154, 187, 223) and numpy RNE on normals
    for v in [1.0, 2.0, 0.5, 1.0 / 127.0, 0.5 / 127.0, -3.75, 65504.0, 6.103515625e-05]:
        h, defect = orc.f32_to_f16(v)
        assert not defect
        assert h == int(np.float32(v).astype(np.float16).view(np.uint16)), v
    rng = np.random.default_rng(7)
    vals = (rng.standard_normal(20000) * np.exp2(rng.integers(-13, 15, 20000))).astype(np.float32)
    vals = vals[(np.abs(vals) >= 2.0 ** -14) & (np.abs(vals) < 65504.0)]
    for v in vals[:4000]:
        h, defect = orc.f32_to_f16(float(v))
        assert not defect
        assert h == int(v.astype(np.float16).view(np.uint16))


def test_f32_to_f16_reference_defects(orc):
    """Documented reference behaviour: f32 subnormals flush to 0 (59-61),
    results below 2^-24 flush to 0 (72-74), and the subnormal-result branch
    (76-77) is reported as the reference defect."""
    assert orc.f32_to_f16(1e-40) == (0, False)
    assert orc.f32_to_f16(1e-9) == (0, False)
    _, defect = orc.f32_to_f16(1e-6)   # 2^-19.9: subnormal in binary16, the reference traps
    assert defect == 1
    assert orc.f32_to_f16(1e6)[0] == 0x7C00


# ---- gguf.zig block arithmetic (gguf.zig:567-586) ----

def test_block_sizes_and_tensor_bytes(orc):
    lib = orc.lib()
    assert lib.orc_block_size(orc.IQ2_XXS) == 256 and lib.orc_block_bytes(orc.IQ2_XXS) == 66
    assert lib.orc_block_size(orc.F32) == 1 and lib.orc_block_bytes(orc.F32) == 4
    assert lib.orc_block_size(orc.Q8_0) == 32 and lib.orc_block_bytes(orc.Q8_0) == 34
    assert orc.tensor_bytes(orc.IQ2_XXS, 256) == 66
    assert orc.tensor_bytes(orc.F32, 4) == 16
    # config shapes
    assert orc.tensor_bytes(orc.Q8_0, 1536 * 2048) == 3342336
    assert orc.tensor_bytes(orc.IQ2_XXS, 1536 * 2048) == 811008


# ---- IQ2_XXS tables ----

def test_ksigns_closed_form(orc):
    for c in range(128):
        s = orc.ksigns(c)
        assert s & 0x7F == c
        assert bin(s).count("1") % 2 == 0  # even number of negative signs


def test_grid_invariants(orc):
    g = [orc.grid(i) for i in range(256)]
    assert len(set(g)) == 256 and g == sorted(g)
    for v in g:
        assert set(v.to_bytes(8, "little")) <= {8, 25, 43}
    assert g[0] == 0x0808080808080808
    assert g[1] == 0x080808080808082B


def _reference_text():
    path = os.path.join(REFERENCE_SRC, "dequant.zig")
    if not os.path.exists(path):
        pytest.skip("reference sources not present (build container only)")
    return open(path).read()


def test_tables_match_reference_literals(orc):
    src = _reference_text()
    start = src.index("pub const iq2xxs_grid")
    grid = [int(v, 16) for v in re.findall(r"0x[0-9a-fA-F]{16}", src[start:src.index("};", start)])]
    assert grid == [orc.grid(i) for i in range(256)]
    start = src.index("pub const ksigns_iq2xs")
    ks = [int(v) for v in re.findall(r"\d+", src[src.index("{", start):src.index("}", start)])]
    assert ks == [orc.ksigns(i) for i in range(128)]


# ---- dequantisation ----

def test_dequant_q8_0_closed_form_all_scales(orc):
    """Every f16 scale code with a fixed qs pattern: out = f32(d) * q exactly."""
    codes = np.arange(65536, dtype=np.uint32)
    q = ((np.arange(32) * 37) % 255 - 127).astype(np.int8)
    blocks = np.empty((65536, 34), dtype=np.uint8)
    blocks[:, 0:2] = codes.astype(np.uint16).view(np.uint8).reshape(-1, 2)
    blocks[:, 2:] = np.broadcast_to(q.view(np.uint8), (65536, 32))
    got = orc.dequantize(blocks.reshape(-1), orc.Q8_0, 65536 * 32).reshape(65536, 32)
    d = codes.astype(np.uint16).view(np.float16).astype(np.float32)
    with np.errstate(invalid="ignore"):
        ref = d[:, None] * q.astype(np.float32)[None, :]
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def _iq2_block(d_bits, aux0, aux1):
    """One superblock from per-sub-block (aux0, aux1) u32 pairs."""
    b = np.zeros(66, dtype=np.uint8)
    b[0:2] = np.array([d_bits], dtype=np.uint16).view(np.uint8)
    words = np.zeros(16, dtype=np.uint32)
    words[0::2] = aux0
    words[1::2] = aux1
    b[2:] = words.view(np.uint8)
    return b


def test_iq2_all_zero_block_is_one(orc):
    # d = 1.0, every index 0 (all bytes 8), ls = 0 -> 1.0 * 0.5 * 0.25 * 8 = 1.0
    out = orc.dequantize(_iq2_block(0x3C00, np.zeros(8, np.uint32), np.zeros(8, np.uint32)), orc.IQ2_XXS, 256)
    assert np.all(out == 1.0)


def test_iq2_byte_order_sign_bits_and_scale(orc):
    """Hand-derived from the format: grid index 1 = 0x080808080808082b puts 43
    in column 0 (little-endian); sign code 1 -> ksigns 0x81 negates columns 0
    and 7; ls = 15 gives db = d * 15.5 / 4; group l uses byte l of aux0 and
    bits 7l..7l+6 of aux1."""
    aux0 = np.zeros(8, np.uint32)
    aux1 = np.zeros(8, np.uint32)
    aux0[0] = 1                      # group 0 of sub-block 0 -> index 1
    aux1[0] = 1                      # sign code 1 for group 0
    aux0[3] = 1 << 16                # sub-block 3, group 2 -> index 1
    aux1[3] = (3 << 14) | (15 << 28)  # sub-block 3, group 2 sign code 3, ls 15
    out = orc.dequantize(_iq2_block(0x3C00, aux0, aux1), orc.IQ2_XXS, 256)
    db0 = 0.125
    exp0 = np.full(8, 8 * db0, np.float32)
    exp0[0] = 43 * db0
    exp0[0] *= -1
    exp0[7] *= -1
    assert np.array_equal(out[0:8], exp0)
    assert np.all(out[8:32] == 1.0)
    db3 = 15.5 / 4
    g = out[96 + 16:96 + 24]
    exp3 = np.full(8, 8 * db3, np.float32)
    exp3[0] = 43 * db3
    exp3[0] *= -1   # code 3 -> bits 0, 1 set, parity even -> bit 7 clear
    exp3[1] *= -1
    assert np.array_equal(g, exp3)
    assert np.all(out[96:112] == np.float32(8 * db3))


def test_iq2_brute_force_one_group(orc):
    """Every grid index x sign code x ls for one 8-weight group, against the
    format definition evaluated from the codebook bytes."""
    idx = np.arange(256 * 128 * 16, dtype=np.uint32) % 256
    code = (np.arange(256 * 128 * 16, dtype=np.uint32) // 256) % 128
    ls = np.arange(256 * 128 * 16, dtype=np.uint32) // (256 * 128)
    n = idx.size
    blocks = np.zeros((n, 66), dtype=np.uint8)
    blocks[:, 0:2] = np.array([0x3555], np.uint16).view(np.uint8)  # d = 0.333...
    words = np.zeros((n, 16), dtype=np.uint32)
    words[:, 0] = idx
    words[:, 1] = code | (ls << 28)
    blocks[:, 2:] = words.view(np.uint8)
    out = orc.dequantize(blocks.reshape(-1), orc.IQ2_XXS, n * 256).reshape(n, 256)[:, :8]
    d = np.float32(np.array([0x3555], np.uint16).view(np.float16)[0])
    db = (d * (np.float32(0.5) + ls.astype(np.float32))) * np.float32(0.25)
    grid = np.array([orc.grid(i) for i in range(256)], dtype=np.uint64)
    mags = ((grid[idx][:, None] >> (8 * np.arange(8, dtype=np.uint64))) & 0xFF).astype(np.float32)
    neg = ((code[:, None] >> np.arange(7)) & 1).astype(bool)
    parity = (np.array([bin(c).count("1") for c in range(128)])[code] & 1).astype(bool)
    neg = np.concatenate([neg, parity[:, None]], axis=1)
    ref = (db[:, None] * mags) * np.where(neg, np.float32(-1), np.float32(1))
    assert np.array_equal(out.view(np.uint32), ref.astype(np.float32).view(np.uint32))
