"""GGUF files through the library's native reader (include/fuel_rocm.h,
frq_gguf_*): the header of fuel_formats::gguf::Content (fuel-formats/src/
gguf.rs:378-461) read over a memory map, and tensors uploaded verbatim as
quantized storages (QuantizedDeviceKernels::load_quantized).

    g = GgufFile(path)
    g.metadata["llama.block_count"]     # python value (ints, floats, bool, str, nested lists)
    g.tensors["blk.0.attn_q.weight"]    # TensorInfo(dtype, dims, offset, nbytes)
    qs = g.load_quantized(dev, "blk.0.attn_q.weight")
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from ._native import check, lib

# ValueType codes (gguf.rs:125-143)
VT_U8, VT_I8, VT_U16, VT_I16, VT_U32, VT_I32, VT_F32, VT_BOOL, VT_STRING, VT_ARRAY, VT_U64, VT_I64, VT_F64 = range(13)
_UNSIGNED = (VT_U8, VT_U16, VT_U32, VT_U64)
_SIGNED = (VT_I8, VT_I16, VT_I32, VT_I64)


@dataclass(frozen=True)
class TensorInfo:
    dtype: int            # GgmlDType code
    dims: tuple           # outermost first (fuel's Shape order)
    offset: int           # relative to tensor_data_offset
    nbytes: int           # elem_count / block_size * type_size


@dataclass(frozen=True)
class Value:
    """A metadata value with its GGUF type (the Value enum)."""
    type: int
    value: object


def _value(v: C.c_void_p) -> Value:
    L = lib()
    t = L.frq_gguf_value_type(v)
    if t == VT_STRING:
        s, n = C.c_char_p(), C.c_size_t()
        check(L.frq_gguf_value_string(v, C.byref(s), C.byref(n)))
        return Value(t, C.string_at(s, n.value).decode("utf-8"))
    if t == VT_ARRAY:
        n = C.c_size_t()
        check(L.frq_gguf_value_array(v, C.byref(n)))
        items = []
        for j in range(n.value):
            e = C.c_void_p()
            check(L.frq_gguf_value_array_at(v, j, C.byref(e)))
            items.append(_value(e))
        return Value(t, items)
    u, i, f = C.c_uint64(), C.c_int64(), C.c_double()
    check(L.frq_gguf_value_scalar(v, C.byref(u), C.byref(i), C.byref(f)))
    if t == VT_BOOL:
        return Value(t, bool(u.value))
    if t in _UNSIGNED:
        return Value(t, int(u.value))
    if t in _SIGNED:
        return Value(t, int(i.value))
    return Value(t, float(f.value))


def plain(v: Value):
    """A Value as plain python data (lists for arrays)."""
    return [plain(e) for e in v.value] if v.type == VT_ARRAY else v.value


class GgufFile:
    def __init__(self, path: str):
        L = lib()
        h = C.c_void_p()
        check(L.frq_gguf_open(str(path).encode(), C.byref(h)))
        self._h = h
        self.path = str(path)
        self.version = int(L.frq_gguf_version(h))
        self.tensor_data_offset = int(L.frq_gguf_tensor_data_offset(h))
        self.values: dict[str, Value] = {}
        for i in range(L.frq_gguf_meta_count(h)):
            key, v = C.c_char_p(), C.c_void_p()
            check(L.frq_gguf_meta_at(h, i, C.byref(key), C.byref(v)))
            self.values[key.value.decode("utf-8")] = _value(v)
        self.metadata = {k: plain(v) for k, v in self.values.items()}
        self.tensors: dict[str, TensorInfo] = {}
        self._index: dict[str, int] = {}
        dims = (C.c_uint64 * 16)()
        for i in range(L.frq_gguf_tensor_count(h)):
            name, dt, nd, off, nb = C.c_char_p(), C.c_int(), C.c_size_t(), C.c_uint64(), C.c_uint64()
            check(L.frq_gguf_tensor_info(h, i, C.byref(name), C.byref(dt), C.byref(nd), dims, 16, C.byref(off),
                                         C.byref(nb)))
            key = name.value.decode("utf-8")
            self.tensors[key] = TensorInfo(int(dt.value), tuple(int(dims[d]) for d in range(nd.value)),
                                           int(off.value), int(nb.value))
            self._index[key] = i

    def close(self) -> None:
        if self._h:
            lib().frq_gguf_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _find(self, name: str) -> int:
        idx = C.c_size_t()
        check(lib().frq_gguf_find_tensor(self._h, name.encode(), C.byref(idx)))
        return idx.value

    def tensor_bytes(self, name: str) -> np.ndarray:
        """A copy of the tensor's bytes (uint8) out of the mapping."""
        p, n = C.c_void_p(), C.c_uint64()
        check(lib().frq_gguf_tensor_data(self._h, self._find(name), C.byref(p), C.byref(n)))
        return np.frombuffer(C.string_at(p, n.value), np.uint8).copy()

    def copy_to_device(self, dev, name: str, dst_ptr: int) -> int:
        """Copy the tensor's bytes from the mapping to device address dst_ptr
        (no host copy); returns the byte count."""
        p, n = C.c_void_p(), C.c_uint64()
        check(lib().frq_gguf_tensor_data(self._h, self._find(name), C.byref(p), C.byref(n)))
        check(lib().frq_memcpy_htod(dev.handle, C.c_void_p(dst_ptr), p, n.value))
        return n.value

    def load_quantized(self, dev, name: str):
        """load_quantized of the tensor's blocks into a new device storage."""
        from .backend import RocmQStorage

        h = C.c_void_p()
        check(lib().frq_gguf_load_quantized(dev.handle, self._h, self._find(name), C.byref(h)))
        return RocmQStorage(dev, h)
