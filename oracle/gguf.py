"""GGUF reader and writer in plain Python: test infrastructure (the checker of
the library's native reader and the maker of test files), never product code.

`read` restates fuel_formats::gguf::Content::read (fuel-formats/src/
gguf.rs:378-461) with VersionedMagic::read (:44-58), read_string (:70-85),
ValueType::from_u32 (:125-143) and Value::read (:305-347); tensor byte
lengths follow the lazy loaders (fuel-core/src/lazy_quantized_llama.rs:
251-260).  `write` lays a file out the same way (Value::write and
write_string, gguf.rs:87-92 and :349-375, for the values).

Pinned by tests/test_gguf.py against byte strings assembled field by field
with struct.pack in the test itself (known answers for every value type,
versions 1-3, alignment rules, repeated keys, string cleanup and each error).
"""
from __future__ import annotations

import struct
from dataclasses import dataclass, field

DEFAULT_ALIGNMENT = 32
(VT_U8, VT_I8, VT_U16, VT_I16, VT_U32, VT_I32, VT_F32, VT_BOOL, VT_STRING, VT_ARRAY,
 VT_U64, VT_I64, VT_F64) = range(13)
_SCALAR = {VT_U8: "<B", VT_I8: "<b", VT_U16: "<H", VT_I16: "<h", VT_U32: "<I", VT_I32: "<i",
           VT_F32: "<f", VT_U64: "<Q", VT_I64: "<q", VT_F64: "<d"}
# GgmlDType::from_u32 codes -> (block_size, type_size)  (fuel-ir/src/quantized.rs:36-104)
DTYPES = {0: (1, 4), 1: (1, 2), 30: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24),
          8: (32, 34), 9: (32, 36), 10: (256, 84), 11: (256, 110), 12: (256, 144), 13: (256, 176),
          14: (256, 210), 15: (256, 292)}


class GgufError(ValueError):
    pass


@dataclass
class Value:
    type: int
    value: object  # int / float / bool / str / list[Value]


def plain(v: Value):
    return [plain(e) for e in v.value] if v.type == VT_ARRAY else v.value


@dataclass
class TensorInfo:
    dtype: int
    dims: tuple      # outermost first
    offset: int
    nbytes: int


@dataclass
class Content:
    version: int
    metadata: dict = field(default_factory=dict)   # key -> Value (insertion order = first appearance)
    tensors: dict = field(default_factory=dict)    # name -> TensorInfo
    tensor_data_offset: int = 0


class _R:
    def __init__(self, b: bytes):
        self.b, self.pos, self.version = b, 0, 0

    def take(self, n: int) -> bytes:
        if len(self.b) - self.pos < n:
            raise GgufError("gguf: unexpected end of file")
        out = self.b[self.pos:self.pos + n]
        self.pos += n
        return out

    def unpack(self, fmt: str):
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def count(self) -> int:
        return self.unpack("<I") if self.version == 1 else self.unpack("<Q")

    def string(self) -> str:
        raw = self.take(self.count())
        raw = raw.rstrip(b"\0")  # trailing NULs only
        return raw.decode("utf-8", errors="replace")

    def value_type(self) -> int:
        t = self.unpack("<I")
        if t > 12:
            raise GgufError(f"unrecognized value-type {t:#08x}")
        return t

    def value(self, t: int) -> Value:
        if t in _SCALAR:
            return Value(t, self.unpack(_SCALAR[t]))
        if t == VT_BOOL:
            b = self.unpack("<B")
            if b > 1:
                raise GgufError(f"unexpected bool value {b}")
            return Value(t, bool(b))
        if t == VT_STRING:
            return Value(t, self.string())
        et = self.value_type()
        n = self.count()
        return Value(t, [self.value(et) for _ in range(n)])


def read(data: bytes) -> Content:
    r = _R(data)
    magic = r.unpack("<I")
    if magic not in (0x46554747, 0x47475546):
        raise GgufError(f"unknown magic 0x{magic:08x}")
    version = r.unpack("<I")
    if version not in (1, 2, 3):
        raise GgufError(f"gguf: unsupported magic/version Gguf/{version}")
    r.version = version
    c = Content(version)
    n_tensors, n_kv = r.count(), r.count()
    for _ in range(n_kv):
        key = r.string()
        c.metadata[key] = r.value(r.value_type())
    for _ in range(n_tensors):
        name = r.string()
        nd = r.unpack("<I")
        dims = [r.count() for _ in range(nd)][::-1]
        dt = r.unpack("<I")
        if dt not in DTYPES:
            raise GgufError(f"unknown dtype for tensor {dt}")
        off = r.unpack("<Q")
        elems = 1
        for d in dims:
            elems *= d
        bs, ts = DTYPES[dt]
        c.tensors[name] = TensorInfo(dt, tuple(dims), off, elems // bs * ts)
    align = DEFAULT_ALIGNMENT
    a = c.metadata.get("general.alignment")
    if a is not None:
        if a.type in (VT_U8, VT_U16, VT_U32) or (a.type in (VT_I8, VT_I16, VT_I32) and a.value >= 0):
            align = a.value
    if align == 0:
        raise GgufError("gguf: general.alignment is 0")
    c.tensor_data_offset = (r.pos + align - 1) // align * align
    return c


# ---- writer ----

def _w_string(s, version: int) -> bytes:
    raw = s.encode("utf-8") if isinstance(s, str) else bytes(s)
    return (struct.pack("<I", len(raw)) if version == 1 else struct.pack("<Q", len(raw))) + raw


def _w_value(v: Value, version: int) -> bytes:
    if v.type in _SCALAR:
        return struct.pack(_SCALAR[v.type], v.value)
    if v.type == VT_BOOL:
        return struct.pack("<B", int(v.value))
    if v.type == VT_STRING:
        return _w_string(v.value, version)
    et = v.value[0].type if v.value else VT_U32
    n = struct.pack("<I", len(v.value)) if version == 1 else struct.pack("<Q", len(v.value))
    return struct.pack("<I", et) + n + b"".join(_w_value(e, version) for e in v.value)


def write(metadata: list, tensors: list, version: int = 3, alignment: int = DEFAULT_ALIGNMENT) -> bytes:
    """metadata: [(key, Value)]; tensors: [(name, dtype, dims outermost first,
    data bytes)].  Tensor data are placed in order, each at an offset rounded
    up to `alignment`, after the header padded to `alignment` (pass the same
    value as any general.alignment entry)."""
    cnt = (lambda n: struct.pack("<I", n)) if version == 1 else (lambda n: struct.pack("<Q", n))
    out = bytearray(struct.pack("<II", 0x46554747, version))
    out += cnt(len(tensors)) + cnt(len(metadata))
    for key, v in metadata:
        out += _w_string(key, version) + struct.pack("<I", v.type) + _w_value(v, version)
    offs, off = [], 0
    for _, _, _, data in tensors:
        off = (off + alignment - 1) // alignment * alignment
        offs.append(off)
        off += len(data)
    for (name, dt, dims, _), o in zip(tensors, offs):
        out += _w_string(name, version) + struct.pack("<I", len(dims))
        for d in reversed(dims):
            out += struct.pack("<I", d) if version == 1 else struct.pack("<Q", d)
        out += struct.pack("<IQ", dt, o)
    start = (len(out) + alignment - 1) // alignment * alignment
    out += b"\0" * (start - len(out))
    for (_, _, _, data), o in zip(tensors, offs):
        out += b"\0" * (start + o - len(out))
        out += bytes(data)
    return bytes(out)
