"""A minimal GGUF writer for the reader's tests. It is written from the GGUF
file format, not from the library.

Layout (little-endian):
  - magic, then the u32 version;
  - the tensor count and the metadata count;
  - the metadata entries: key string, u32 value type, value;
  - the tensor infos: name string, u32 n_dims, ne[0..n_dims) (innermost
    first), u32 ggml type, u64 offset relative to the data section;
  - padding to the alignment, then the tensor data.

Version 1 writes counts, string / array lengths and dims as u32. Versions 2
and 3 write them as u64.

The writer places the data section where [ext] candle-core 0.11
gguf_file::Content::read looks for it. That is the next multiple of
general.alignment when the value is a U8/U16/U32 or a non-negative
I8/I16/I32, else of 32. The engine's loader reads files through Content
(engine/src/model.rs:535).
"""
from __future__ import annotations

import struct

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q",
        I64: "<q", F64: "<d"}


class _W:
    def __init__(self, version: int):
        self.v1 = version == 1
        self.buf = bytearray()

    def u32(self, v):
        self.buf += struct.pack("<I", v)

    def u64(self, v):
        self.buf += struct.pack("<Q", v)

    def length(self, n):
        (self.u32 if self.v1 else self.u64)(n)

    def string(self, s):
        b = s if isinstance(s, (bytes, bytearray)) else s.encode()
        self.length(len(b))
        self.buf += b

    def value(self, t, v):
        if t == STRING:
            self.string(v)
        elif t == ARRAY:
            et, items = v
            self.u32(et)
            self.length(len(items))
            for it in items:
                self.value(et, it)
        else:
            self.buf += struct.pack(_FMT[t], v)


def effective_alignment(kv) -> int:
    """Content::read's alignment: the last general.alignment entry if it is
    an unsigned or non-negative signed integer of at most 32 bits, else 32."""
    align = 32
    for key, t, v in kv:
        k = key if isinstance(key, str) else key.decode("utf-8", "replace")
        if k == "general.alignment":
            align = v if (t in (U8, U16, U32) or (t in (I8, I16, I32) and v >= 0)) else 32
    return align


def build(kv, tensors, version: int = 3, magic: bytes = b"GGUF", data_align: int | None = None):
    """kv: [(key, type, value)]. tensors: [(name, ggml_type, shape
    row-major, data bytes)] or (..., data, rel_offset) to force an offset.
    Returns (file bytes, data section start, [relative offsets])."""
    w = _W(version)
    w.buf += magic
    w.u32(version)
    w.length(len(tensors))
    w.length(len(kv))
    for key, t, v in kv:
        w.string(key)
        w.u32(t)
        w.value(t, v)
    align = data_align or effective_alignment(kv)
    offs, cur = [], 0
    for tt in tensors:
        data = tt[3]
        if len(tt) > 4:
            offs.append(tt[4])
        else:
            offs.append(cur)
            cur += len(data)
            cur = (cur + align - 1) // align * align
    for tt, off in zip(tensors, offs):
        name, gt, shape = tt[0], tt[1], tt[2]
        w.string(name)
        w.u32(len(shape))
        for d in reversed(shape):  # ne[0] is the innermost (row length)
            (w.u32 if w.v1 else w.u64)(d)
        w.u32(gt)
        w.u64(off)
    start = (len(w.buf) + align - 1) // align * align
    out = bytearray(w.buf) + bytes(start - len(w.buf))
    for tt, off in zip(tensors, offs):
        data = bytes(tt[3])
        end = start + off + len(data)
        if len(out) < end:
            out += bytes(end - len(out))
        out[start + off:end] = data
    return bytes(out), start, offs
