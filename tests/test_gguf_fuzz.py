"""Bounded fuzz of the GGUF parser (mmhip_gguf_open and the getters) over
mutated files: a valid file from tests/gguf_writer.py with every metadata
value type, arrays and tensors, then seeded mutations (bit flips, bytes set to
0x00 / 0xFF / 0x7F, a random 8-byte length field, truncation, a duplicated
span). Every file must either be rejected with an error code or parse into
values that every getter reads without leaving the mapping. The run stops at
the first failure (an unexpected exception, or, under the sanitizer build,
any invalid read). The parser's own bounds checks are what is tested; the
reference's parser (gguf.zig:266-413) reads with read(2) and has no such
checks to compare with."""
import ctypes
import os
import struct

import numpy as np
import pytest

import gguf_writer as gw
import mmhip as mm

N_CASES = int(os.environ.get("MMHIP_FUZZ_CASES", "5000"))

META = [
    ("general.architecture", gw.STRING, "deepseek2"),
    ("general.alignment", gw.U32, 32),
    ("a.u8", gw.U8, 7), ("a.i16", gw.I16, -2), ("a.u32", gw.U32, 123456), ("a.f32", gw.F32, 0.25),
    ("a.bool", gw.BOOL, False), ("a.str", gw.STRING, "hello"), ("a.u64", gw.U64, 2 ** 33),
    ("a.i64", gw.I64, -9), ("a.f64", gw.F64, 2.5),
    ("a.arr_i32", gw.ARRAY, (gw.I32, [1, -2, 3])),
    ("a.arr_str", gw.ARRAY, (gw.STRING, ["x", "yz", ""])),
    ("deepseek2.expert_weights_scale", gw.F32, 1.5),
]


def _base():
    rng = np.random.default_rng(77)
    tensors = [
        ("t.f32", [5, 2], mm.F32, rng.normal(size=(2, 5)).astype(np.float32)),
        ("t.q8", [64, 2], mm.Q8_0, mm.make_weight(rng, mm.Q8_0, 2, 64)),
        ("t.iq2", [256, 1, 2], mm.IQ2_XXS, mm.make_weight(rng, mm.IQ2_XXS, 1, 256, 2)),
    ]
    return gw.build(META, tensors)[0]


def _mutate(rng, blob):
    b = bytearray(blob)
    kind = int(rng.integers(0, 7))
    n = len(b)
    if kind == 0:  # flip 1-4 bits
        for _ in range(int(rng.integers(1, 5))):
            i = int(rng.integers(0, n))
            b[i] ^= 1 << int(rng.integers(0, 8))
    elif kind == 1:  # special byte values
        for _ in range(int(rng.integers(1, 4))):
            b[int(rng.integers(0, n))] = int(rng.choice([0x00, 0xFF, 0x7F, 0x80]))
    elif kind == 2:  # a random 8-byte little-endian value (length / count / offset fields)
        i = int(rng.integers(0, max(1, n - 8)))
        vals = [0, 1, 2 ** 31, 2 ** 32 + 5, 2 ** 63, 2 ** 64 - 1, int(rng.integers(0, 2 ** 20))]
        v = vals[int(rng.integers(0, len(vals)))]
        b[i:i + 8] = struct.pack("<Q", v)
    elif kind == 3:  # truncate
        del b[int(rng.integers(0, n)):]
    elif kind == 4:  # duplicate a span
        i = int(rng.integers(0, n))
        j = min(n, i + int(rng.integers(1, 64)))
        b[i:i] = b[i:j]
    elif kind == 5:  # a random 4-byte value (type ids, dims counts)
        i = int(rng.integers(0, max(1, n - 4)))
        vals = [0, 3, 12, 13, 31, 255, 2 ** 31, 2 ** 32 - 1]
        b[i:i + 4] = struct.pack("<I", vals[int(rng.integers(0, len(vals)))])
    else:  # delete a span
        i = int(rng.integers(0, n))
        del b[i:i + int(rng.integers(1, 32))]
    return bytes(b)


def _exercise(g):
    info = g.info()
    assert info["version"] == 3
    for t in g.tensors():
        assert t["n_dims"] <= 4
        if t["data"] and t["n_bytes"]:
            # every byte the descriptor promises, read through the mapping
            np.ctypeslib.as_array(ctypes.cast(t["data"], ctypes.POINTER(ctypes.c_uint8)), (t["n_bytes"],)).sum()
        g.tensor(t["name"])  # names may hold any bytes (a NUL ends the C string)
    for k in g.keys():
        g.meta_type(k)
        g.meta_int(k)
        g.meta_float(k)
        g.meta_string(k)
        g.meta_array(k)
    g.meta_int("no.such.key")


def test_fuzz_mutated_files(tmp_path):
    mm.load_library()
    base = _base()
    p = tmp_path / "f.gguf"
    p.write_bytes(base)
    with mm.Gguf(p) as g:  # the unmutated file parses
        _exercise(g)
    rng = np.random.default_rng(2024)
    opened = rejected = 0
    for case in range(N_CASES):
        blob = _mutate(rng, base)
        if rng.random() < 0.3:
            blob = _mutate(rng, blob)
        p.write_bytes(blob)
        try:
            g = mm.Gguf(p)
        except mm.MmhipError:
            rejected += 1
            continue
        try:
            _exercise(g)
            opened += 1
        except mm.MmhipError:
            opened += 1
        except Exception as e:  # the first failure stops the run, with its case
            pytest.fail(f"case {case}: {type(e).__name__}: {e}")
        finally:
            g.close()
    print(f"\n{N_CASES} mutated files: {opened} opened and read, {rejected} rejected")
    assert opened > 0 and rejected > 0
