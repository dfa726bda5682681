"""A small GGUF v3 writer for the tests (the file layout of
crates/strata-gguf/src/reader.rs:1-12): header, typed metadata, tensor
directory, padding to the alignment, payloads. `raw_*` hooks let a test
write malformed files byte by byte."""
from __future__ import annotations

import struct

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "B", I8: "b", U16: "H", I16: "h", U32: "I", I32: "i", F32: "f", BOOL: "B", U64: "Q", I64: "q",
        F64: "d"}


def gstr(s) -> bytes:
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def payload(ty: int, v) -> bytes:
    """A value's bytes without its type tag (array items carry none)."""
    if ty == STRING:
        return gstr(v)
    if ty == ARRAY:
        elem, items = v
        return struct.pack("<IQ", elem, len(items)) + b"".join(payload(elem, it) for it in items)
    return struct.pack("<" + _FMT[ty], v)


class Writer:
    def __init__(self, alignment: int = 32, version: int = 3, magic: int = 0x46554747):
        self.kvs = []
        self.infos = []
        self.blobs = []
        self.offset = 0
        self.alignment = alignment
        self.version = version
        self.magic = magic

    def kv(self, key, ty: int, v):
        self.kvs.append(gstr(key) + struct.pack("<I", ty) + payload(ty, v))
        return self

    def raw_kv(self, b: bytes):
        self.kvs.append(b)
        return self

    def tensor(self, name, shape, ty: int, data: bytes, offset=None, pad_to: int = 32):
        off = self.offset if offset is None else offset
        self.infos.append(gstr(name) + struct.pack("<I", len(shape)) + b"".join(struct.pack("<Q", d) for d in shape)
                          + struct.pack("<IQ", ty, off))
        if offset is None:
            blob = bytes(data)
            pad = (-len(blob)) % pad_to
            self.blobs.append(blob + b"\0" * pad)
            self.offset += len(blob) + pad
        return self

    def raw_info(self, b: bytes):
        self.infos.append(b)
        return self

    def finish(self, truncate_data: int = 0) -> bytes:
        head = struct.pack("<IIQQ", self.magic, self.version, len(self.infos), len(self.kvs))
        body = head + b"".join(self.kvs) + b"".join(self.infos)
        body += b"\0" * ((-len(body)) % self.alignment)
        data = b"".join(self.blobs)
        if truncate_data:
            data = data[:-truncate_data]
        return body + data
