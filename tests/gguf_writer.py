"""A small GGUF v3 writer for test files, written from the published GGUF
layout (ggml's docs/gguf.md): header (magic, version, tensor count, metadata
count), metadata key/value records, tensor descriptors, padding to the
alignment, then the tensor data with every tensor starting at an aligned
offset. Values are given as (type, value); arrays as (ARRAY, (elem_type,
[values])). The parser under test never reads this module."""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?", U64: "<Q",
        I64: "<q", F64: "<d"}


def gguf_string(s) -> bytes:
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def encode_value(vtype, value) -> bytes:
    if vtype in _FMT:
        return struct.pack(_FMT[vtype], value)
    if vtype == STRING:
        return gguf_string(value)
    if vtype == ARRAY:
        et, items = value
        return struct.pack("<IQ", et, len(items)) + b"".join(encode_value(et, v) for v in items)
    raise ValueError(vtype)


def header(n_tensors, n_kv, magic=b"GGUF", version=3) -> bytes:
    return magic + struct.pack("<IQQ", version, n_tensors, n_kv)


def kv(key, vtype, value) -> bytes:
    return gguf_string(key) + struct.pack("<I", vtype) + encode_value(vtype, value)


def tensor_info(name, dims, ggml_type, offset) -> bytes:
    return gguf_string(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims) + \
        struct.pack("<IQ", ggml_type, offset)


def build(meta, tensors, alignment=32):
    """meta: [(key, type, value)]; tensors: [(name, dims, ggml_type, bytes)].
    Returns (file bytes, data offset, per-tensor offsets within the data)."""
    blobs = [np.ascontiguousarray(data).view(np.uint8).reshape(-1).tobytes() for _, _, _, data in tensors]
    offsets, pos = [], 0
    for b in blobs:
        pos += (-pos) % alignment
        offsets.append(pos)
        pos += len(b)
    out = bytearray(header(len(tensors), len(meta)))
    for key, vt, v in meta:
        out += kv(key, vt, v)
    for (name, dims, gt, _), off in zip(tensors, offsets):
        out += tensor_info(name, dims, gt, off)
    data_offset = len(out) + (-len(out)) % alignment
    out += b"\0" * (data_offset - len(out))
    for b, off in zip(blobs, offsets):
        assert len(out) <= data_offset + off
        out += b"\0" * (data_offset + off - len(out))
        out += b
    return bytes(out), data_offset, offsets


def write(path, meta, tensors, alignment=32):
    blob, data_offset, offsets = build(meta, tensors, alignment)
    with open(path, "wb") as f:
        f.write(blob)
    return data_offset, offsets
