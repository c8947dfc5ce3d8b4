"""Minimal GGUF v3 writer for the tests (test infrastructure, not the product).

Layout, little-endian, as the reference's loader reads it
(src/loader/gguf_loader.cpp:36-91, 245-436, 474-497, 540-590):
  magic u32 "GGUF", version u32, tensor count u64, metadata count u64;
  metadata: key (u64 length + bytes), value type u32, value;
  inventory: name, n_dims u32, ne u64 x n_dims, ggml type u32, offset u64
  (relative to the data start); data start = header end rounded up to the
  alignment (32, or general.alignment); each tensor's data aligned likewise.
"""
from __future__ import annotations

import struct

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
           U64: "<Q", I64: "<q", F64: "<d"}


def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, v) -> bytes:
    if vtype == STR:
        return _str(v)
    if vtype == ARR:
        etype, items = v
        out = struct.pack("<IQ", etype, len(items))
        for it in items:
            out += _value(etype, it)
        return out
    return struct.pack(_SCALAR[vtype], v)


def gguf_bytes(kv: list, tensors: list, version: int = 3, alignment: int = 32, magic: int = 0x46554747) -> bytes:
    """kv: [(key, type, value)], value of ARR = (elem_type, [items]).
    tensors: [(name, ggml_type, ne tuple, data bytes)]."""
    head = struct.pack("<IIQQ", magic, version, len(tensors), len(kv))
    for key, vtype, v in kv:
        head += _str(key) + struct.pack("<I", vtype) + _value(vtype, v)
    offsets, off = [], 0
    for _, _, _, data in tensors:
        offsets.append(off)
        off += len(data)
        off = (off + alignment - 1) // alignment * alignment
    for (name, gtype, ne, _), o in zip(tensors, offsets):
        head += _str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", n) for n in ne)
        head += struct.pack("<IQ", gtype, o)
    pad = (-len(head)) % alignment
    blob = bytearray(head + b"\0" * pad)
    data_start = len(blob)
    for (_, _, _, data), o in zip(tensors, offsets):
        need = data_start + o - len(blob)
        blob += b"\0" * need
        blob += data
    return bytes(blob)


def write_gguf(path: str, kv: list, tensors: list, **kw) -> int:
    """Writes the file; returns its bytes."""
    b = gguf_bytes(kv, tensors, **kw)
    with open(path, "wb") as f:
        f.write(b)
    return b
