"""Minimal GGUF v3 writer for tests (test infrastructure).

Byte layout of GGUF v3 as the reference reads it (src/gguf.rs:108-237 and its
tests' helpers, src/gguf/tests.rs:28-39): "GGUF", version 3, tensor count,
metadata count, metadata (key string, u32 type, value), tensor infos (name,
u32 rank, u64 dims, u32 type, u64 offset), padding to general.alignment
(default 32), then the tensor data at the recorded offsets.
"""
import struct

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B",
        U64: "<Q", I64: "<q", F64: "<d"}


def string(s) -> bytes:
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def value(kind: int, v) -> bytes:
    if kind == STRING:
        return string(v)
    if kind == ARRAY:
        elem, items = v
        out = struct.pack("<IQ", elem, len(items))
        return out + b"".join(value(elem, x) for x in items)
    return struct.pack(_FMT[kind], v)


def header(tensors: int, metadata: int) -> bytes:
    return b"GGUF" + struct.pack("<IQQ", 3, tensors, metadata)


def build(metadata=(), tensors=(), alignment: int = 32, data_pad: int = 0) -> bytes:
    """metadata: [(key, kind, value)]; tensors: [(name, shape, type_code, payload bytes)].
    Tensor data is laid out in order, each at the next multiple of `alignment`."""
    out = bytearray(header(len(tensors), len(metadata)))
    for key, kind, v in metadata:
        out += string(key) + struct.pack("<I", kind) + value(kind, v)
    offsets, pos = [], 0
    for _, _, _, payload in tensors:
        pos = (pos + alignment - 1) // alignment * alignment
        offsets.append(pos)
        pos += len(payload)
    for (name, shape, code, _), off in zip(tensors, offsets):
        out += string(name) + struct.pack("<I", len(shape)) + b"".join(struct.pack("<Q", d) for d in shape)
        out += struct.pack("<IQ", code, off)
    if not tensors:  # no data section
        return bytes(out) + bytes(data_pad)
    start = (len(out) + alignment - 1) // alignment * alignment
    out += bytes(start - len(out))
    for (_, _, _, payload), off in zip(tensors, offsets):
        out += bytes(start + off - len(out))
        out += payload
    out += bytes(data_pad)
    return bytes(out)
