"""Python mirror of fuel's quantized seams over the C ABI.

* ``RocmDevice``   -- ``DynBackendDevice`` + ``QuantizedDeviceKernels``
  (fuel-backend-contract/src/quantized.rs:108-119: ``qzeros``, ``load_quantized``).
* ``RocmStorage``  -- a device f32/f16/i32 buffer standing in for ``DynBackendStorage``.
* ``RocmQStorage`` -- ``DynQuantizedStorage`` (quantized.rs:29-103: ``dtype``,
  ``block_size``, ``storage_size_in_bytes``, ``dequantize``, ``dequantize_f16``,
  ``data``, ``device_ptr``, ``fwd``).
* ``qmatmul_f32_rocm_wrapper`` -- the ``KernelRef`` registered at
  ``(OpKind::QMatMul, [F32, U32, F32], Rocm)`` (fuel-dispatch/src/dispatch.rs
  :1638-1718), same argument meaning and error behaviour.

Errors raise ``FuelRocmError`` (fuel's ``Err(Error::Msg(..))``).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import Sequence

import numpy as np

from . import _native as N
from ._native import FuelRocmError, check, lib

_NP = {N.F32: np.float32, N.F16: np.uint16}


def type_size(ggml_dtype: int) -> int:
    return int(lib().frq_type_size(ggml_dtype))


def block_size(ggml_dtype: int) -> int:
    return int(lib().frq_block_size(ggml_dtype))


def device_count() -> int:
    n = C.c_int(0)
    check(lib().frq_device_count(C.byref(n)))
    return n.value


class RocmDevice:
    """One GPU with its own HIP stream and activation workspace."""

    def __init__(self, ordinal: int = 0):
        h = C.c_void_p()
        check(lib().frq_device_open(ordinal, C.byref(h)))
        self._h = h
        self.ordinal = ordinal

    @property
    def handle(self) -> C.c_void_p:
        if self._h is None:
            raise FuelRocmError(N.FRQ_INVALID, "device is closed")
        return self._h

    def close(self) -> None:
        if self._h is not None:
            lib().frq_device_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def synchronize(self) -> None:
        check(lib().frq_sync(self.handle))

    def set_stream(self, hip_stream_ptr: int | None) -> None:
        check(lib().frq_device_set_stream(self.handle, C.c_void_p(hip_stream_ptr or 0)))

    @property
    def cu_count(self) -> int:
        n = C.c_int(0)
        check(lib().frq_device_cu_count(self.handle, C.byref(n)))
        return n.value

    # ---- storages ----
    def alloc(self, shape, dtype=np.float32) -> "RocmStorage":
        return RocmStorage(self, tuple(int(s) for s in np.atleast_1d(shape)), np.dtype(dtype))

    def from_numpy(self, a: np.ndarray) -> "RocmStorage":
        a = np.ascontiguousarray(a)
        s = RocmStorage(self, a.shape, a.dtype)
        s.copy_from(a)
        return s

    # ---- QuantizedDeviceKernels ----
    def qzeros(self, elem_count: int, ggml_dtype: int) -> "RocmQStorage":
        h = C.c_void_p()
        check(lib().frq_qstorage_zeros(self.handle, ggml_dtype, elem_count, C.byref(h)))
        return RocmQStorage(self, h)

    def load_quantized(self, ggml_dtype: int, data) -> "RocmQStorage":
        buf = np.ascontiguousarray(np.frombuffer(memoryview(data).cast("B"), np.uint8))
        h = C.c_void_p()
        check(lib().frq_qstorage_load(self.handle, ggml_dtype, buf.ctypes.data_as(C.c_void_p),
                                      buf.nbytes, C.byref(h)))
        return RocmQStorage(self, h)


class RocmStorage:
    """A contiguous device buffer of `shape` and numpy `dtype`."""

    def __init__(self, dev: RocmDevice, shape: tuple, dtype: np.dtype):
        self.dev = dev
        self.shape = tuple(shape)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape, dtype=np.int64)) * self.dtype.itemsize
        p = C.c_void_p()
        check(lib().frq_malloc(dev.handle, self.nbytes, C.byref(p)))
        self.ptr = p.value or 0

    def free(self) -> None:
        if self.ptr:
            lib().frq_free(self.dev.handle, C.c_void_p(self.ptr))
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def copy_from(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.nbytes == self.nbytes, (a.nbytes, self.nbytes)
        check(lib().frq_memcpy_htod(self.dev.handle, C.c_void_p(self.ptr),
                                    a.ctypes.data_as(C.c_void_p), a.nbytes))

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        check(lib().frq_memcpy_dtoh(self.dev.handle, out.ctypes.data_as(C.c_void_p),
                                    C.c_void_p(self.ptr), self.nbytes))
        return out


class RocmQStorage:
    """``DynQuantizedStorage`` for the ROCm device (block bytes in HBM)."""

    def __init__(self, dev: RocmDevice, handle: C.c_void_p):
        self.dev = dev
        self._h = handle

    def __del__(self):
        try:
            if self._h:
                lib().frq_qstorage_free(self._h)
                self._h = None
        except Exception:
            pass

    @property
    def handle(self):
        return self._h

    def dtype(self) -> int:
        return int(lib().frq_qstorage_dtype(self._h))

    def block_size(self) -> int:
        return int(lib().frq_qstorage_block_size(self._h))

    def storage_size_in_bytes(self) -> int:
        return int(lib().frq_qstorage_size_in_bytes(self._h))

    def data(self) -> bytes:
        n = self.storage_size_in_bytes()
        out = np.empty(n, np.uint8)
        check(lib().frq_qstorage_data(self._h, out.ctypes.data_as(C.c_void_p), n))
        return out.tobytes()

    def device_ptr(self) -> int:
        p = C.c_void_p()
        check(lib().frq_qstorage_device_ptr(self._h, C.byref(p)))
        return p.value or 0

    def dequantize(self, elem_count: int) -> RocmStorage:
        y = self.dev.alloc((elem_count,), np.float32)
        check(lib().frq_qstorage_dequantize(self._h, elem_count, C.c_void_p(y.ptr)))
        return y

    def dequantize_f16(self, elem_count: int) -> RocmStorage:
        y = self.dev.alloc((elem_count,), np.uint16)
        check(lib().frq_qstorage_dequantize_f16(self._h, elem_count, C.c_void_p(y.ptr)))
        return y

    def quantize(self, src: RocmStorage) -> None:
        """from_float of a device f32 source onto this storage (on the device)."""
        if src.dtype != np.float32:
            raise FuelRocmError(N.FRQ_INVALID, f"quantize: expected f32 source, got {src.dtype}")
        check(lib().frq_qstorage_quantize(self._h, C.c_void_p(src.ptr), src.nbytes // 4))

    def quantize_imatrix(self, src: RocmStorage, imatrix_weights, n_per_row: int) -> None:
        """from_float_imatrix of a device f32 source onto this storage
        (quantize_imatrix / quantize_imatrix_onto of the trait seam): Q4_K and
        Q6_K; imatrix_weights is a host sequence of n_per_row f32 weights."""
        if src.dtype != np.float32:
            raise FuelRocmError(N.FRQ_INVALID, f"quantize_imatrix: expected f32 source, got {src.dtype}")
        w = np.ascontiguousarray(imatrix_weights, dtype=np.float32)
        if w.size < n_per_row:
            raise FuelRocmError(N.FRQ_INVALID, f"quantize_imatrix: {w.size} weights for n_per_row={n_per_row}")
        check(lib().frq_qstorage_quantize_imatrix(self._h, C.c_void_p(src.ptr), src.nbytes // 4,
                                                  w.ctypes.data_as(C.c_void_p), n_per_row))

    quantize_imatrix_onto = quantize_imatrix

    def fwd(self, self_shape: Sequence[int], inp: RocmStorage):
        """QMatMul forward: input [..., k] -> fresh output [..., n]
        (fuel-cpu-backend/src/quantized.rs:85-142 semantics): f32 input gives
        f32 output (matmul), f16 input gives f16 output (matmul_f16)."""
        n, k = (int(d) for d in self_shape)
        if inp.dtype not in (np.float32, np.float16):
            raise FuelRocmError(N.FRQ_UNSUPPORTED, "Expected f32/f16")
        if len(inp.shape) < 2:
            raise FuelRocmError(N.FRQ_INVALID, f"input tensor has only one dimension {inp.shape}")
        if inp.shape[-1] != k:
            raise FuelRocmError(N.FRQ_INVALID, f"input tensor {inp.shape} incompatible with {tuple(self_shape)}")
        out_shape = tuple(inp.shape[:-1]) + (n,)
        y = self.dev.alloc(out_shape, inp.dtype)
        m = int(np.prod(inp.shape[:-1]))
        fwd = lib().frq_qstorage_fwd if inp.dtype == np.float32 else lib().frq_qstorage_fwd_f16
        check(fwd(self._h, n, k, C.c_void_p(inp.ptr), m, C.c_void_p(y.ptr)))
        return y, out_shape

    def indexed_moe_forward(self, self_shape: Sequence[int], inp: RocmStorage, ids: RocmStorage):
        """mul_mat_id: self = experts [e, n, k]; input [t, 1 | topk, k] (or
        [t, k]); ids [t, topk] int32 -> fresh output [t, topk, n] with
        y[t, s] = W[ids[t, s]] @ x[t, s or 0]
        (fuel-backend-contract/src/quantized.rs:82-95)."""
        e, n, k = (int(d) for d in self_shape)
        if inp.dtype != np.float32:
            raise FuelRocmError(N.FRQ_UNSUPPORTED, f"indexed_moe_forward: expected f32 input, got {inp.dtype}")
        if ids.dtype != np.int32 or len(ids.shape) != 2:
            raise FuelRocmError(N.FRQ_INVALID, f"indexed_moe_forward: ids must be int32 [t, topk], got "
                                               f"{ids.dtype} {ids.shape}")
        t, topk = ids.shape
        if len(inp.shape) == 2:
            slots = 1
        elif len(inp.shape) == 3:
            slots = inp.shape[1]
        else:
            raise FuelRocmError(N.FRQ_INVALID, f"indexed_moe_forward: input {inp.shape} is not [t, slots, k]")
        if inp.shape[0] != t or inp.shape[-1] != k:
            raise FuelRocmError(N.FRQ_INVALID, f"indexed_moe_forward: input {inp.shape} incompatible with "
                                               f"experts {tuple(self_shape)} and ids {ids.shape}")
        out_shape = (t, topk, n)
        y = self.dev.alloc(out_shape, np.float32)
        check(lib().frq_indexed_moe_forward(self._h, e, n, k, C.c_void_p(inp.ptr), t, slots,
                                            C.c_void_p(ids.ptr), topk, C.c_void_p(y.ptr)))
        return y, out_shape


@dataclass
class QMatMulParams:
    """``OpParams::QMatMul{quant_type, batch_count, m, n, k}`` (fuel-dispatch/src/kernel.rs:482-488);
    quant_type is the GgmlDType code."""

    quant_type: int
    batch_count: int
    m: int
    n: int
    k: int


def qmatmul_f32_rocm_wrapper(inputs: Sequence[RocmStorage], outputs: Sequence[RocmStorage],
                             params: QMatMulParams) -> None:
    """KernelRef for (QMatMul, [F32, U32, F32], Rocm): inputs = [activations f32,
    weight bytes U32-typed], outputs = [pre-allocated f32]; fully overwrites the output."""
    if len(inputs) != 2:
        raise FuelRocmError(N.FRQ_INVALID,
                            f"qmatmul wrapper expects 2 inputs (activations, weight_bytes), got {len(inputs)}")
    if len(outputs) != 1:
        raise FuelRocmError(N.FRQ_INVALID, f"qmatmul wrapper expects 1 output, got {len(outputs)}")
    act, w = inputs
    out = outputs[0]
    if w.dtype != np.uint32:
        raise FuelRocmError(N.FRQ_INVALID,
                            f"qmatmul: weight bytes must be U32-typed (raw block stream), got {w.dtype}")
    p = params
    check(lib().frq_qmatmul(act.dev.handle, p.quant_type, p.batch_count, p.m, p.n, p.k,
                            C.c_void_p(act.ptr), act.nbytes, C.c_void_p(w.ptr), w.nbytes,
                            C.c_void_p(out.ptr), out.nbytes))


# ---- synthetic inputs ----

def fill_normal(dev: RocmDevice, shape, seed: int, stream: int, mean: float = 0.0, std: float = 1.0) -> RocmStorage:
    y = dev.alloc(shape, np.float32)
    check(lib().frq_fill_normal(dev.handle, C.c_void_p(y.ptr), y.nbytes // 4, seed, stream, mean, std))
    return y


def fill_random_bits(dev: RocmDevice, n: int, start: int, seed: int, base: int, stream: int) -> RocmStorage:
    y = dev.alloc((n,), np.uint32)
    check(lib().frq_fill_random_bits(dev.handle, C.c_void_p(y.ptr), n, start, seed, base, stream))
    return y


# ---- parity taps ----

QMM_PATHS = ("matvec", "matvec_multi", "skinny_mfma", "tiled_mfma")


def qmatmul_plan(dev: RocmDevice, ggml_dtype: int, rows: int, n: int, k: int, w_ptr: int, noalloc: bool = False):
    """The kernels frq_qmatmul (or frq_qmatmul_noalloc) runs for this call:
    (path name, tile kernel kind or -1, K splits)."""
    path, kind, ks = C.c_int(), C.c_int(), C.c_int()
    check(lib().frq_qmatmul_plan(dev.handle, ggml_dtype, rows, n, k, C.c_void_p(w_ptr), int(noalloc), C.byref(path),
                                 C.byref(kind), C.byref(ks)))
    return QMM_PATHS[path.value], kind.value, ks.value


def quantize_q8k(dev: RocmDevice, x: RocmStorage, rows: int, k: int) -> np.ndarray:
    """Device BlockQ8K quantization of x [rows, k]; returns the block bytes."""
    out = dev.alloc((rows * (k // 256) * 292,), np.uint8)
    check(lib().frq_quantize_q8k(dev.handle, C.c_void_p(x.ptr), rows, k, C.c_void_p(out.ptr)))
    return out.numpy()


def quantize_q8_0(dev: RocmDevice, x: RocmStorage, rows: int, k: int) -> np.ndarray:
    out = dev.alloc((rows * (k // 32) * 34,), np.uint8)
    check(lib().frq_quantize_q8_0(dev.handle, C.c_void_p(x.ptr), rows, k, C.c_void_p(out.ptr)))
    return out.numpy()


def block_isums(dev: RocmDevice, ggml_dtype: int, w: RocmStorage, x: RocmStorage, m: int, n: int, k: int):
    kb = k // block_size(ggml_dtype)
    isum = dev.alloc((m, n, kb), np.int32)
    msum = dev.alloc((m, n, kb), np.int32)
    check(lib().frq_block_isums(dev.handle, ggml_dtype, m, n, k, C.c_void_p(w.ptr), C.c_void_p(x.ptr),
                                C.c_void_p(isum.ptr), C.c_void_p(msum.ptr)))
    return isum.numpy(), msum.numpy()


def moe_route(dev: RocmDevice, logits: RocmStorage, topk: int):
    """Top-k softmax routing and expert batches of logits [t, e] on the device
    (lazy_nn/moe.rs:90-127, moe_routing.rs:252-275, 334-360).  Returns numpy
    (ids [t, topk], w [t, topk], expert_offsets [e + 1], sorted_token_ids
    [t * topk], sorted_slot [t * topk])."""
    t, e = logits.shape
    ids = dev.alloc((t, topk), np.int32)
    w = dev.alloc((t, topk), np.float32)
    offsets = dev.alloc((e + 1,), np.int32)
    sorted_tok = dev.alloc((t * topk,), np.int32)
    sorted_slot = dev.alloc((t * topk,), np.int32)
    check(lib().frq_moe_route(dev.handle, C.c_void_p(logits.ptr), t, e, topk, C.c_void_p(ids.ptr),
                              C.c_void_p(w.ptr), C.c_void_p(offsets.ptr), C.c_void_p(sorted_tok.ptr),
                              C.c_void_p(sorted_slot.ptr)))
    return ids.numpy(), w.numpy(), offsets.numpy(), sorted_tok.numpy(), sorted_slot.numpy()


def moe_ffn(dev: RocmDevice, ggml_dtype: int, x: RocmStorage, logits: RocmStorage, w_gate, w_up, w_down,
            ffn: int, topk: int, out: RocmStorage | None = None) -> RocmStorage:
    """The quantized expert layer: route logits [t, e], SwiGLU experts over the
    routed rows, weighted combine -> out [t, d] (lazy_nn/moe.rs:296-348).
    w_gate / w_up / w_down: device addresses (int) or RocmQStorage of the
    expert-major block bytes."""
    t, d = x.shape
    e = logits.shape[1]
    if out is None:
        out = dev.alloc((t, d), np.float32)
    ptr = lambda w: w.device_ptr() if isinstance(w, RocmQStorage) else int(w)
    check(lib().frq_moe_ffn(dev.handle, ggml_dtype, t, d, ffn, e, topk, C.c_void_p(x.ptr), C.c_void_p(logits.ptr),
                            C.c_void_p(ptr(w_gate)), C.c_void_p(ptr(w_up)), C.c_void_p(ptr(w_down)),
                            C.c_void_p(out.ptr)))
    return out
