"""A small GGUF writer for the reader's tests.

Writes the published GGUF v2/v3 layout with ``struct`` (little endian):
magic "GGUF", u32 version, u64 tensor count, u64 metadata count; metadata
entries (string key, u32 type, value); tensor infos (string name, u32
n_dims, u64 dims, u32 GGML type, u64 offset from the data section); padding
to the alignment; the tensor bytes.  The reader under test parses the same
layout (GGUFReader.pas:605-745); this writer shares no code with it.
"""
from __future__ import annotations

import struct

# metadata value types
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B",
        U64: "<Q", I64: "<q", F64: "<d"}


def gstr(s) -> bytes:
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def value(t: int, v) -> bytes:
    if t == STR:
        return gstr(v)
    if t == ARR:
        et, items = v
        out = struct.pack("<IQ", et, len(items))
        return out + b"".join(value(et, x) for x in items)
    return struct.pack(_FMT[t], v)


def build(meta, tensors, version: int = 3, alignment: int | None = None, magic: bytes = b"GGUF",
          tensor_count: int | None = None, meta_count: int | None = None):
    """meta: list of (key, type, value); tensors: list of (name, dims, ggml
    type, bytes).  Tensor data is laid out in order, each start padded to the
    alignment (32, or the general.alignment entry's value).

    Returns (file bytes, {name: absolute data offset}).
    """
    align = alignment or 32
    head = magic + struct.pack("<IQQ", version,
                               len(tensors) if tensor_count is None else tensor_count,
                               len(meta) if meta_count is None else meta_count)
    body = b"".join(gstr(k) + struct.pack("<I", t) + value(t, v) for k, t, v in meta)
    rel, off = [], 0
    for _, _, _, data in tensors:
        off = (off + align - 1) // align * align
        rel.append(off)
        off += len(data)
    infos = b""
    for (name, dims, gt, _), r in zip(tensors, rel):
        infos += gstr(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        infos += struct.pack("<IQ", gt, r)
    pre = head + body + infos
    start = (len(pre) + align - 1) // align * align
    blob = bytearray(pre + b"\0" * (start - len(pre)))
    for (_, _, _, data), r in zip(tensors, rel):
        need = start + r
        blob += b"\0" * (need - len(blob))
        blob += data
    return bytes(blob), {t[0]: start + r for t, r in zip(tensors, rel)}
