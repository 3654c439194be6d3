"""fuel_amd -- MI355X (gfx950) quantized-matmul backend for fuel.

The compute path is libfuel_rocm.so (HIP kernels + C ABI, include/fuel_rocm.h);
this package is its Python binding, mirroring fuel's DynQuantizedStorage /
QuantizedDeviceKernels seam and the (QMatMul, [F32, U32, F32]) KernelRef.
"""
from ._native import F16, F32, Q4K, Q6K, Q8K, Q8_0, FuelRocmError, LIB_PATH, SIGNATURES, lib
from .backend import (
    QMatMulParams,
    RocmDevice,
    RocmQStorage,
    RocmStorage,
    block_isums,
    block_size,
    device_count,
    fill_normal,
    fill_random_bits,
    moe_ffn,
    moe_route,
    qmatmul_f32_rocm_wrapper,
    qmatmul_plan,
    quantize_q8_0,
    quantize_q8k,
    type_size,
)
from .gguf import GgufFile

__all__ = [
    "F16", "F32", "Q4K", "Q6K", "Q8K", "Q8_0", "FuelRocmError", "LIB_PATH", "SIGNATURES", "lib",
    "QMatMulParams", "RocmDevice", "RocmQStorage", "RocmStorage", "block_isums", "block_size",
    "device_count", "fill_normal", "fill_random_bits", "moe_ffn", "moe_route",
    "qmatmul_f32_rocm_wrapper", "qmatmul_plan", "quantize_q8_0", "quantize_q8k", "type_size", "GgufFile",
]
