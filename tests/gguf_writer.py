"""Minimal GGUF v3 writer for tests (little endian; the layout the reader
parses: header, metadata, tensor infos, data section at `alignment`)."""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q",
           I64: "<q", F64: "<d"}


def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(vtype, v):
    if vtype == STRING:
        return _str(v)
    if vtype == ARRAY:
        etype, items = v
        out = struct.pack("<IQ", etype, len(items))
        return out + b"".join(_value(etype, x) for x in items)
    return struct.pack(_SCALAR[vtype], v)


def gguf_bytes(metadata, tensors, alignment=32, version=3, magic=b"GGUF", pad_data=True):
    """metadata: [(key, vtype, value)]; tensors: [(name, ggml_type, shape (ne0 first), bytes)].
    Tensor data are placed in order, each at a multiple of `alignment` within the data section."""
    out = bytearray(magic + struct.pack("<IQQ", version, len(tensors), len(metadata)))
    for k, t, v in metadata:
        out += _str(k) + struct.pack("<I", t) + _value(t, v)
    offs, off = [], 0
    for name, gt, shape, data in tensors:
        offs.append(off)
        off += len(data)
        off = (off + alignment - 1) // alignment * alignment
    for (name, gt, shape, data), o in zip(tensors, offs):
        out += _str(name) + struct.pack("<I", len(shape)) + b"".join(struct.pack("<Q", d) for d in shape)
        out += struct.pack("<IQ", gt, o)
    out += b"\0" * ((-len(out)) % alignment)
    base = len(out)
    for (name, gt, shape, data), o in zip(tensors, offs):
        out += b"\0" * (base + o - len(out))
        out += bytes(data)
    if pad_data:
        out += b"\0" * ((-len(out)) % alignment)
    return bytes(out)


def write(path, metadata, tensors, **kw):
    with open(path, "wb") as f:
        f.write(gguf_bytes(metadata, tensors, **kw))


def q8_rows(blocks: np.ndarray, n_rows: int):
    """GGUF Q8_0 bytes of n_rows rows (already row-major bytes)."""
    b = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1)
    assert b.size % n_rows == 0
    return b
