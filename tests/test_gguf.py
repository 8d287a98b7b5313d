"""GGUF v3 parsing through the C ABI (gguf.zig:266-413, model.zig:261-269),
host only: files written by tests/gguf_writer.py from the published layout
are read back, value by value; malformed files fail with the reference's
error names (gguf.zig:270-276, 303, 446-447, 466-467, 527-528, 536). Block
sizes follow the reference's tests (gguf.zig:566-586)."""
import struct

import numpy as np
import pytest

import gguf_writer as gw
import mmhip as mm

META = [
    ("general.architecture", gw.STRING, "deepseek2"),
    ("t.u8", gw.U8, 200), ("t.i8", gw.I8, -5), ("t.u16", gw.U16, 60000), ("t.i16", gw.I16, -30000),
    ("t.u32", gw.U32, 4000000000), ("t.i32", gw.I32, -7), ("t.f32", gw.F32, 0.1), ("t.bool", gw.BOOL, True),
    ("t.str", gw.STRING, "GLM-4.7 µ"), ("t.u64", gw.U64, 2 ** 40 + 3), ("t.i64", gw.I64, -2 ** 40),
    ("t.f64", gw.F64, -1.0 / 3.0),
    ("t.arr_u32", gw.ARRAY, (gw.U32, [1, 2, 0xFFFFFFFF])),
    ("t.arr_f32", gw.ARRAY, (gw.F32, [0.5, -2.0])),
    ("t.arr_str", gw.ARRAY, (gw.STRING, ["a", "", "tokén"])),
    ("t.arr_empty", gw.ARRAY, (gw.I8, [])),
    ("deepseek2.expert_weights_scale", gw.F32, 1.8),
]


def _tensors(rng):
    return [
        ("output_norm.weight", [7], mm.F32, rng.normal(size=7).astype(np.float32)),
        ("blk.0.ffn_gate_inp.weight", [40, 3], mm.F32, rng.normal(size=(3, 40)).astype(np.float32)),
        ("blk.0.attn_q_a.weight", [64, 3], mm.Q8_0, mm.make_weight(rng, mm.Q8_0, 3, 64)),
        ("blk.1.ffn_gate_exps.weight", [256, 2, 4], mm.IQ2_XXS, mm.make_weight(rng, mm.IQ2_XXS, 2, 256, 4)),
        ("blk.1.ffn_gate_inp.weight", [5, 2], mm.F16, mm.make_weight(rng, mm.F16, 2, 5)),
    ]


@pytest.fixture(scope="module")
def lib():
    return mm.load_library()


def _open_bytes(tmp_path, blob, name="f.gguf"):
    p = tmp_path / name
    p.write_bytes(blob)
    return mm.Gguf(p)


def test_block_sizes_kat(orc):
    """gguf.zig:566-586: IQ2_XXS 256 / 66, F32 1 / 4, Q8_0 32 / 34; tensorBytes(256) = 66, F32 tensorBytes(4) = 16."""
    assert mm.tensor_bytes(mm.IQ2_XXS, 1, 256) == 66
    assert mm.tensor_bytes(mm.F32, 1, 4) == 16
    assert mm.tensor_bytes(mm.Q8_0, 1, 32) == 34


def test_round_trip(tmp_path, lib):
    rng = np.random.default_rng(5)
    tensors = _tensors(rng)
    data_offset, offsets = gw.write(tmp_path / "m.gguf", META, tensors)
    with mm.Gguf(tmp_path / "m.gguf") as g:
        info = g.info()
        assert info["version"] == 3 and info["tensor_count"] == 5 and info["metadata_count"] == len(META)
        assert info["alignment"] == 32 and info["data_offset"] == data_offset and data_offset % 32 == 0
        assert g.keys() == [k for k, _, _ in META]
        ints = {"t.u8": 200, "t.i8": -5, "t.u16": 60000, "t.i16": -30000, "t.u32": 4000000000, "t.i32": -7,
                "t.u64": 2 ** 40 + 3, "t.i64": -2 ** 40}
        for k, v in ints.items():
            assert g.meta_int(k) == v, k
        assert g.meta_int("t.f32") is None and g.meta_int("t.bool") is None and g.meta_int("nope") is None
        assert g.meta_float("t.f32") == float(np.float32(0.1))
        assert g.meta_float("t.f64") == -1.0 / 3.0
        assert g.meta_float("t.i32") is None
        assert g.meta_string("t.str") == "GLM-4.7 µ".encode()
        assert g.meta_string("t.u8") is None
        assert g.meta_type("t.bool") == gw.BOOL and g.meta_type("t.arr_str") == gw.ARRAY
        assert g.meta_array("t.arr_u32") == (gw.U32, 3, struct.pack("<3I", 1, 2, 0xFFFFFFFF))
        assert g.meta_array("t.arr_f32") == (gw.F32, 2, struct.pack("<2f", 0.5, -2.0))
        assert g.meta_array("t.arr_str") == (gw.STRING, 3, b"".join(gw.gguf_string(s) for s in
                                                                    ["a", "", "tokén"]))
        assert g.meta_array("t.arr_empty") == (gw.I8, 0, b"")
        listed = g.tensors()
        assert [t["name"] for t in listed] == [t[0] for t in tensors]
        for (name, dims, gt, data), off, t in zip(tensors, offsets, listed):
            assert t == g.tensor(name)
            assert t["n_dims"] == len(dims) and t["dims"] == tuple(dims + [1] * (4 - len(dims)))
            assert t["type"] == gt and t["offset"] == off
            assert t["n_elements"] == int(np.prod(dims))
            assert t["n_bytes"] == data.nbytes
            assert np.array_equal(g.tensor_bytes(name), np.ascontiguousarray(data).view(np.uint8).reshape(-1))
        assert g.tensor("blk.9.ffn_up_exps.weight") is None


@pytest.mark.parametrize("vtype", [gw.U32, gw.U64])
def test_alignment_key(tmp_path, lib, vtype):
    rng = np.random.default_rng(6)
    meta = [("general.alignment", vtype, 64)] + META[:3]
    tensors = _tensors(rng)
    data_offset, offsets = gw.write(tmp_path / "a.gguf", meta, tensors, alignment=64)
    with mm.Gguf(tmp_path / "a.gguf") as g:
        assert g.info()["alignment"] == 64 and g.info()["data_offset"] == data_offset
        assert data_offset % 64 == 0
        name, _, _, data = tensors[3]
        assert np.array_equal(g.tensor_bytes(name), data.view(np.uint8).reshape(-1))


def test_alignment_other_type_ignored(tmp_path, lib):
    """Only a u32 or u64 general.alignment counts (gguf.zig:340-346)."""
    meta = [("general.alignment", gw.I32, 64)]
    blob, data_offset, _ = gw.build(meta, [("x", [4], mm.F32, np.ones(4, np.float32))], alignment=32)
    with _open_bytes(tmp_path, blob) as g:
        assert g.info()["alignment"] == 32 and g.info()["data_offset"] == data_offset


def test_repeated_key_and_tensor(tmp_path, lib):
    meta = [("k", gw.U32, 1), ("j", gw.U32, 2), ("k", gw.U32, 3)]
    x, y = np.arange(4, dtype=np.float32), np.arange(8, dtype=np.float32)
    blob, _, _ = gw.build(meta, [("w", [4], mm.F32, x), ("w", [8], mm.F32, y)])
    with _open_bytes(tmp_path, blob) as g:
        assert g.keys() == ["k", "j"] and g.meta_int("k") == 3
        assert g.info()["tensor_count"] == 2 and g.info()["n_tensors"] == 1
        assert g.tensor("w")["dims"][0] == 8
        assert np.array_equal(g.tensor_bytes("w").view(np.float32), y)


def _expect_error(tmp_path, blob, text, code=-2):
    with pytest.raises(mm.MmhipError) as e:
        _open_bytes(tmp_path, blob)
    assert text in str(e.value) and e.value.code == code, str(e.value)


def test_errors(tmp_path, lib):
    good, _, _ = gw.build(META[:2], [("x", [4], mm.F32, np.ones(4, np.float32))])
    _expect_error(tmp_path, b"GGUX" + good[4:], "InvalidMagic")
    _expect_error(tmp_path, gw.header(0, 0, version=2), "UnsupportedVersion 2")
    _expect_error(tmp_path, gw.header(0, 1) + gw.gguf_string("k") + struct.pack("<I", 13), "UnsupportedMetadataType",
                  code=-3)
    _expect_error(tmp_path, gw.header(0, 1) + gw.gguf_string("k") + struct.pack("<IIQ", gw.ARRAY, gw.ARRAY, 1),
                  "UnsupportedArrayType", code=-3)
    _expect_error(tmp_path, gw.header(0, 1) + struct.pack("<Q", 65537) + b"k" * 65537, "StringTooLong")
    _expect_error(tmp_path, gw.header(0, 1) + gw.kv("k", gw.STRING, "x" * 65536)[:-1], "EndOfStream")
    _expect_error(tmp_path, gw.header(0, 1) + gw.gguf_string("k") + struct.pack("<IIQ", gw.ARRAY, gw.U8, 10000001),
                  "ArrayTooLong")
    _expect_error(tmp_path, gw.header(1, 0) + gw.gguf_string("t") + struct.pack("<I", 5) + b"\1" * 40,
                  "TooManyDimensions")
    _expect_error(tmp_path, gw.header(0, 1) + gw.kv("general.alignment", gw.U32, 0), "alignment is 0")
    # Every proper prefix of a good file's header part is a truncated stream.
    head = len(gw.header(1, 2)) + sum(len(gw.kv(*m)) for m in META[:2]) + len(gw.tensor_info("x", [4], 0, 0))
    for cut in sorted({1, 3, 4, 8, 23, 24, 30, head // 2, head - 1}):
        _expect_error(tmp_path, good[:cut], "EndOfStream")
    with pytest.raises(mm.MmhipError):
        mm.Gguf(tmp_path / "missing.gguf")
    for bad in (tmp_path, tmp_path / "empty.gguf"):
        if bad != tmp_path:
            bad.write_bytes(b"")
        with pytest.raises(mm.MmhipError) as e:
            mm.Gguf(bad)
        assert "regular file" in str(e.value) and e.value.code == -2


def test_data_outside_file_has_no_pointer(tmp_path, lib):
    blob, _, _ = gw.build([], [("x", [64], mm.F32, np.ones(64, np.float32))])
    with _open_bytes(tmp_path, blob[:-4]) as g:
        t = g.tensor("x")
        assert t["n_bytes"] == 256 and not t["data"]
    blob = gw.header(1, 0) + gw.tensor_info("q", [32], 3, 0)  # Q4_1: not read by this library
    with _open_bytes(tmp_path, blob + b"\0" * 64) as g:
        t = g.tensor("q")
        assert t["type"] == 3 and t["n_bytes"] == 0 and not t["data"]


def test_u64_too_large_for_int(tmp_path, lib):
    blob, _, _ = gw.build([("big", gw.U64, 2 ** 63)], [])
    with _open_bytes(tmp_path, blob) as g:
        with pytest.raises(mm.MmhipError):
            g.meta_int("big")


def test_overflowing_dims_have_no_pointer(tmp_path, lib):
    blob = gw.header(1, 0) + gw.tensor_info("w", [2 ** 33, 2 ** 33, 4], mm.Q8_0, 0)
    with _open_bytes(tmp_path, blob + b"\0" * 64) as g:
        t = g.tensor("w")
        assert t["n_elements"] == 0 and t["n_bytes"] == 0 and not t["data"]
