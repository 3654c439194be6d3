"""ctypes binding of libfuel_rocm.so (the C ABI in include/fuel_rocm.h).

There is no fallback: if the HIP library is missing or fails to load, every
entry point raises.  Build it with ``make -C fuel_amd`` (or
``__graft_entry__.build()``).
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libfuel_rocm.so")

FRQ_OK, FRQ_MISALIGNED, FRQ_INVALID, FRQ_UNSUPPORTED, FRQ_WORKSPACE, FRQ_INTERNAL = range(6)
STATUS_NAMES = {
    FRQ_MISALIGNED: "misaligned",
    FRQ_INVALID: "invalid problem",
    FRQ_UNSUPPORTED: "unsupported",
    FRQ_WORKSPACE: "workspace",
    FRQ_INTERNAL: "internal",
}

# GgmlDType codes (fuel-ir/src/quantized.rs:36-76)
F32, F16, Q8_0, Q4K, Q6K, Q8K = 0, 1, 8, 12, 14, 15


class FuelRocmError(RuntimeError):
    """A failed call; mirrors fuel_ir::Error::Msg carrying the backend message."""

    def __init__(self, status: int, msg: str):
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {msg}")
        self.status = status


# Every exported symbol of include/fuel_rocm.h with its ctypes signature.
_vp, _sz, _i32 = C.c_void_p, C.c_size_t, C.c_int
SIGNATURES = {
    "frq_last_error": (C.c_char_p, []),
    "frq_type_size": (_sz, [_i32]),
    "frq_block_size": (_sz, [_i32]),
    "frq_device_count": (_i32, [C.POINTER(C.c_int)]),
    "frq_device_open": (_i32, [_i32, C.POINTER(_vp)]),
    "frq_device_close": (_i32, [_vp]),
    "frq_device_set_stream": (_i32, [_vp, _vp]),
    "frq_sync": (_i32, [_vp]),
    "frq_device_cu_count": (_i32, [_vp, C.POINTER(C.c_int)]),
    "frq_device_workspace_bytes": (_i32, [_vp, C.POINTER(_sz)]),
    "frq_malloc": (_i32, [_vp, _sz, C.POINTER(_vp)]),
    "frq_free": (_i32, [_vp, _vp]),
    "frq_memcpy_htod": (_i32, [_vp, _vp, _vp, _sz]),
    "frq_memcpy_dtoh": (_i32, [_vp, _vp, _vp, _sz]),
    "frq_memcpy_dtod": (_i32, [_vp, _vp, _vp, _sz]),
    "frq_memset": (_i32, [_vp, _vp, _i32, _sz]),
    "frq_qstorage_zeros": (_i32, [_vp, _i32, _sz, C.POINTER(_vp)]),
    "frq_qstorage_load": (_i32, [_vp, _i32, _vp, _sz, C.POINTER(_vp)]),
    "frq_qstorage_free": (_i32, [_vp]),
    "frq_qstorage_dtype": (_i32, [_vp]),
    "frq_qstorage_block_size": (_sz, [_vp]),
    "frq_qstorage_size_in_bytes": (_sz, [_vp]),
    "frq_qstorage_data": (_i32, [_vp, _vp, _sz]),
    "frq_qstorage_device_ptr": (_i32, [_vp, C.POINTER(_vp)]),
    "frq_qstorage_dequantize": (_i32, [_vp, _sz, _vp]),
    "frq_qstorage_dequantize_f16": (_i32, [_vp, _sz, _vp]),
    "frq_qstorage_quantize": (_i32, [_vp, _vp, _sz]),
    "frq_qstorage_quantize_imatrix": (_i32, [_vp, _vp, _sz, _vp, _sz]),
    "frq_qstorage_fwd": (_i32, [_vp, _sz, _sz, _vp, _sz, _vp]),
    "frq_qstorage_fwd_f16": (_i32, [_vp, _sz, _sz, _vp, _sz, _vp]),
    "frq_qmatmul": (_i32, [_vp, _i32, _sz, _sz, _sz, _sz, _vp, _sz, _vp, _sz, _vp, _sz]),
    "frq_qmatmul_noalloc": (_i32, [_vp, _i32, _sz, _sz, _sz, _sz, _vp, _sz, _vp, _sz, _vp, _sz]),
    "frq_qmatmul_plan": (_i32, [_vp, _i32, _sz, _sz, _sz, _vp, _i32, C.POINTER(C.c_int), C.POINTER(C.c_int),
                                C.POINTER(C.c_int)]),
    "frq_quantize_q8k": (_i32, [_vp, _vp, _sz, _sz, _vp]),
    "frq_quantize_q8_0": (_i32, [_vp, _vp, _sz, _sz, _vp]),
    "frq_moe_route": (_i32, [_vp, _vp, _sz, _sz, _sz, _vp, _vp, _vp, _vp, _vp]),
    "frq_indexed_moe_forward": (_i32, [_vp, _sz, _sz, _sz, _vp, _sz, _sz, _vp, _sz, _vp]),
    "frq_moe_ffn": (_i32, [_vp, _i32, _sz, _sz, _sz, _sz, _sz, _vp, _vp, _vp, _vp, _vp, _vp]),
    "frq_qmatmul_fused": (_i32, [_vp, _i32, _sz, _sz, _sz, _vp, _vp, _sz, _vp, _vp, C.c_float, _i32, _vp, _sz]),
    "frq_qmatmul_fused_pair": (_i32, [_vp, _sz, _sz, _vp, _sz, _vp, C.c_float, _i32, _sz, _vp, _vp, _i32, _sz, _vp,
                                      _vp]),
    "frq_qmatmul_fused_glu": (_i32, [_vp, _i32, _sz, _sz, _sz, _vp, _vp, _vp, _sz, _vp, C.c_float, _vp, _sz]),
    "frq_attention_decode_workspace": (_sz, [_sz, _sz]),
    "frq_attention_decode": (_i32, [_vp, _sz, _sz, _sz, _vp, _vp, _vp, _vp, _vp, _vp, _vp, C.c_float, _vp, _sz,
                                    _vp]),
    "frq_attention_decode_oproj": (_i32, [_vp, _sz, _sz, _sz, _vp, _vp, _vp, _vp, _vp, _vp, _vp, C.c_float, _vp,
                                          _sz, _i32, _vp, _sz, _vp]),
    "frq_argmax_embed": (_i32, [_vp, _vp, _sz, _vp, _sz, _vp, _sz, _vp, _vp, _vp]),
    "frq_rms_norm_rows": (_i32, [_vp, _sz, _sz, _vp, _sz, _vp, C.c_float, _vp, _sz]),
    "frq_rope_append_rows": (_i32, [_vp, _sz, _sz, _sz, _sz, _vp, _sz, _vp, _sz, _vp, _vp, _sz, _vp, _vp]),
    "frq_attention_prefill": (_i32, [_vp, _sz, _sz, _sz, _sz, _vp, _sz, _vp, _vp, _sz, C.c_float, _vp, _sz]),
    "frq_swiglu_rows": (_i32, [_vp, _sz, _sz, _vp, _sz, _vp, _sz]),
    "frq_add": (_i32, [_vp, _sz, _vp, _vp]),
    "frq_gather_rows": (_i32, [_vp, _vp, _sz, _sz, _vp, _sz, _vp]),
    "frq_block_isums": (_i32, [_vp, _i32, _sz, _sz, _sz, _vp, _vp, _vp, _vp]),
    "frq_fill_random_bits": (_i32, [_vp, _vp, _sz, C.c_uint64, C.c_uint64, C.c_uint32, C.c_uint32]),
    "frq_fill_normal": (_i32, [_vp, _vp, _sz, C.c_uint64, C.c_uint32, C.c_float, C.c_float]),
    "frq_probe_read": (_i32, [_vp, _vp, _sz, _i32, _i32, _i32, _vp]),
    "frq_gguf_open": (_i32, [C.c_char_p, _vp]),
    "frq_gguf_close": (_i32, [_vp]),
    "frq_gguf_version": (_i32, [_vp]),
    "frq_gguf_tensor_data_offset": (C.c_uint64, [_vp]),
    "frq_gguf_tensor_count": (_sz, [_vp]),
    "frq_gguf_tensor_info": (_i32, [_vp, _sz, _vp, _vp, _vp, _vp, _sz, _vp, _vp]),
    "frq_gguf_find_tensor": (_i32, [_vp, C.c_char_p, _vp]),
    "frq_gguf_tensor_data": (_i32, [_vp, _sz, _vp, _vp]),
    "frq_gguf_load_quantized": (_i32, [_vp, _vp, _sz, _vp]),
    "frq_gguf_meta_count": (_sz, [_vp]),
    "frq_gguf_meta_at": (_i32, [_vp, _sz, _vp, _vp]),
    "frq_gguf_meta_find": (_i32, [_vp, C.c_char_p, _vp]),
    "frq_gguf_value_type": (_i32, [_vp]),
    "frq_gguf_value_scalar": (_i32, [_vp, _vp, _vp, _vp]),
    "frq_gguf_value_u64": (_i32, [_vp, _vp]),
    "frq_gguf_value_string": (_i32, [_vp, _vp, _vp]),
    "frq_gguf_value_array": (_i32, [_vp, _vp]),
    "frq_gguf_value_array_at": (_i32, [_vp, _sz, _vp]),
}

_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is not built; run `make -C {HERE}` (the HIP path has no CPU fallback)"
            )
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(status: int) -> None:
    if status != FRQ_OK:
        raise FuelRocmError(status, lib().frq_last_error().decode(errors="replace"))
