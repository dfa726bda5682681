"""A plain-Python restatement of the reference's GGUF v3 reader.

TEST INFRASTRUCTURE ONLY: the tests parse the same bytes with this and with
the library's reader and compare every field. It follows
crates/strata-gguf/src/reader.rs:22-445 and metadata.rs:1-111 step for step:

* header: magic "GGUF" (reader.rs:22,258-261), version 3 only (:262-265),
  tensor and kv counts (u64);
* metadata (:123-176): strings of at most 65,535 bytes that must be UTF-8
  (:99-114), value types 0..12, arrays of at most 2^24 items whose items
  are parsed in full up to 2^20 and only the first 64 beyond (:159-172),
  at most two nested array levels (:124-127); a repeated key keeps the last
  value (HashMap insert);
* directory (:276-310): unique names (a duplicate is an error), 1..4 dims;
* alignment (:312-319): general.alignment when MetaValue::as_int gives a
  positive value (an integer type; a u64 value's int field is 0, so it does
  not count), else 32; data_start = directory end rounded up; past the end
  of the file an error if there are tensors, else clamped (:321-336);
* tensor_payload_bytes (:399-423): product of dims (a zero or overflowing
  dim is Truncated) // block size * block bytes, from quant.rs:125-164;
* tensor_data (:425-445): bounds-checked against the file.
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field

MAGIC = 0x46554747
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)

# quant.rs:125-164: type id -> (block elements, block bytes)
GEOMETRY = {
    0: (1, 4), 1: (1, 2), 30: (1, 2), 24: (1, 1),
    2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34), 9: (32, 36), 20: (32, 18), 39: (32, 17),
    10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210), 16: (256, 66),
    17: (256, 74), 18: (256, 98), 21: (256, 110), 22: (256, 82), 23: (256, 136), 29: (256, 56),
    40: (64, 36), 41: (128, 18), 42: (64, 18),
}


class GgufError(Exception):
    def __init__(self, kind: str, msg: str = ""):
        super().__init__(f"{kind}: {msg}")
        self.kind = kind  # io, format, truncated, unsupported_quant


@dataclass
class Meta:
    ty: int
    int: int = 0
    uint: int = 0
    float: float = 0.0
    string: str = ""
    elem: int = U32
    count: int = 0

    def as_int(self):
        # metadata.rs:90-96: integer types give their int field (u64: 0)
        if self.ty not in (STRING, ARRAY, F32, F64):
            return self.int
        return None

    def as_float(self):
        if self.ty in (STRING, ARRAY):
            return None
        return self.float if self.ty in (F32, F64) else float(self.int)

    def as_str(self):
        return self.string if self.ty == STRING else None


@dataclass
class Tensor:
    name: str
    shape: list
    ty: int
    offset: int


@dataclass
class GgufFile:
    version: int
    alignment: int
    data_start: int
    size: int
    n_kv: int
    meta: dict = field(default_factory=dict)
    tensors: list = field(default_factory=list)
    data: bytes = b""

    def find(self, name):
        for i, t in enumerate(self.tensors):
            if t.name == name:
                return i
        return None

    def payload_bytes(self, t: Tensor) -> int:
        if not t.shape:
            raise GgufError("format", "no dims")
        if t.ty not in GEOMETRY:
            raise GgufError("unsupported_quant", f"type {t.ty}")
        block, size = GEOMETRY[t.ty]
        n = 1
        for d in t.shape:
            if d == 0 or n > (2**64 - 1) // d:
                raise GgufError("truncated", "zero or overflowing dim")
            n *= d
        nb = (n // block) * size
        if nb >= 2**64:
            raise GgufError("truncated", "payload overflows")
        return nb

    def tensor_data(self, t: Tensor) -> bytes:
        nb = self.payload_bytes(t)
        start = self.data_start + t.offset
        end = start + nb
        if start >= 2**64 or end >= 2**64 or end > self.size:
            raise GgufError("truncated", f"{t.name}: past the end")
        return self.data[start:end]


class _Cursor:
    def __init__(self, data: bytes):
        self.d = data
        self.pos = 0

    def take(self, n: int) -> bytes:
        if n > len(self.d) - self.pos:
            raise GgufError("truncated", f"expected {n}, found {len(self.d) - self.pos}")
        b = self.d[self.pos:self.pos + n]
        self.pos += n
        return b

    def unpack(self, fmt: str):
        return struct.unpack("<" + fmt, self.take(struct.calcsize("<" + fmt)))[0]

    def string(self) -> str:
        n = self.unpack("Q")
        if n > 65535:
            raise GgufError("format", f"bad key length {n}")
        raw = self.take(n)
        try:
            return raw.decode("utf-8", errors="strict")
        except UnicodeDecodeError as e:
            raise GgufError("format", "string not UTF-8") from e

    def value(self, ty: int, depth: int) -> Meta:
        if depth > 2:
            raise GgufError("format", "bad value type 9")
        v = Meta(ty)
        if ty in (U8, I8, U16, I16, U32, I32):
            v.int = self.unpack("BbHhIi"[ty])
        elif ty == F32:
            v.float = float(self.unpack("f"))
        elif ty == BOOL:
            v.int = int(self.unpack("B") != 0)
        elif ty == STRING:
            v.string = self.string()
        elif ty == U64:
            v.uint = self.unpack("Q")
        elif ty == I64:
            v.int = self.unpack("q")
        elif ty == F64:
            v.float = self.unpack("d")
        elif ty == ARRAY:
            elem = self.unpack("I")
            if elem > F64:
                raise GgufError("format", f"bad value type {elem}")
            count = self.unpack("Q")
            if count > 1 << 24:
                raise GgufError("format", "bad value type 9")
            v.elem, v.count = elem, count
            keep = count if count <= 1 << 20 else 64
            for _ in range(keep):
                self.value(elem, depth + 1)
        else:
            raise GgufError("format", f"bad value type {ty}")
        return v


def parse(data: bytes) -> GgufFile:
    c = _Cursor(data)
    magic = c.unpack("I")
    if magic != MAGIC:
        raise GgufError("format", f"bad magic {magic:#x}")
    version = c.unpack("I")
    if version != 3:
        raise GgufError("format", f"unsupported version {version}")
    n_tensors = c.unpack("Q")
    n_kv = c.unpack("Q")
    meta = {}
    for _ in range(n_kv):
        key = c.string()
        ty = c.unpack("I")
        if ty > F64:
            raise GgufError("format", f"bad value type {ty}")
        meta[key] = c.value(ty, 0)
    tensors, names = [], set()
    for _ in range(n_tensors):
        name = c.string()
        if name in names:
            raise GgufError("format", f"duplicate tensor {name}")
        names.add(name)
        nd = c.unpack("I")
        if nd == 0 or nd > 4:
            raise GgufError("format", f"{nd} dims")
        shape = [c.unpack("Q") for _ in range(nd)]
        ty = c.unpack("I")
        offset = c.unpack("Q")
        tensors.append(Tensor(name, shape, ty, offset))
    align = 32
    a = meta.get("general.alignment")
    if a is not None and a.as_int() is not None and a.as_int() > 0:
        align = a.as_int()
    start = -(-c.pos // align) * align
    if start > len(data):
        if tensors:
            raise GgufError("truncated", f"data starts at {start}, file has {len(data)}")
        start = len(data)
    return GgufFile(version, align, start, len(data), n_kv, meta, tensors, data)


def open_file(path: str) -> GgufFile:
    try:
        with open(path, "rb") as f:
            data = f.read()
    except OSError as e:
        raise GgufError("io", str(e)) from e
    return parse(data)


def split_paths(any_path: str) -> list:
    """reader.rs:524-572."""
    import os
    at = any_path.rfind("-of-")
    if at < 0 or at < 6 or any_path[at - 6] != "-" or len(any_path) != at + 14 or any_path[at + 9:at + 14] != ".gguf":
        return [any_path]
    a, b = any_path[at - 5:at], any_path[at + 4:at + 9]
    if not (a.isascii() and a.isdigit() and b.isascii() and b.isdigit()):
        return [any_path]
    no, n = int(a), int(b)
    if n < 1 or no < 1 or no > n:
        return [any_path]
    out = []
    for i in range(1, n + 1):
        p = any_path[:at - 5] + f"{i:05d}" + any_path[at:]
        if not os.path.exists(p):
            raise GgufError("io", f"{p}: missing model shard {i} of {n}")
        out.append(p)
    return out
