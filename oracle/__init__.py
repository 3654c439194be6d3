"""ctypes front-end of the CPU oracle (oracle/fuel_oracle.c).

TEST INFRASTRUCTURE ONLY: the checker for the HIP path and the source of the
CPU baseline.  Only tests/, ``__graft_entry__.smoke()`` and bench.py's
``cpu_baseline`` leg import this package.  The product (fuel_amd/) never does.

Block dtypes below are byte-exact with the reference's ``#[repr(C)]`` structs
(fuel-quantized/src/k_quants.rs:92-169).
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# (FUEL_ORACLE_LIB: another build of the same source, e.g. the sanitizer run's)
LIB_PATH = os.environ.get("FUEL_ORACLE_LIB") or os.path.join(HERE, "build", "libfuel_oracle.so")

# GgmlDType codes (fuel-ir/src/quantized.rs:36-76)
Q8_0, Q4K, Q6K, Q8K = 8, 12, 14, 15

BLOCK_Q8_0 = np.dtype([("d", "<u2"), ("qs", "i1", 32)])
BLOCK_Q4K = np.dtype([("d", "<u2"), ("dmin", "<u2"), ("scales", "u1", 12), ("qs", "u1", 128)])
BLOCK_Q6K = np.dtype([("ql", "u1", 128), ("qh", "u1", 64), ("scales", "i1", 16), ("d", "<u2")])
BLOCK_Q8K = np.dtype([("d", "<f4"), ("qs", "i1", 256), ("bsums", "<i2", 16)])
BLOCK_DTYPE = {Q8_0: BLOCK_Q8_0, Q4K: BLOCK_Q4K, Q6K: BLOCK_Q6K, Q8K: BLOCK_Q8K}
BLOCK_SIZE = {Q8_0: 32, Q4K: 256, Q6K: 256, Q8K: 256}
TYPE_SIZE = {Q8_0: 34, Q4K: 144, Q6K: 210, Q8K: 292}
VEC_DOT_TYPE = {Q8_0: Q8_0, Q4K: Q8K, Q6K: Q8K}

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        vp, sz, f32, i32, u32, u64 = C.c_void_p, C.c_size_t, C.c_float, C.c_int, C.c_uint32, C.c_uint64
        sigs = {
            "fo_type_size": (sz, [i32]),
            "fo_block_size": (sz, [i32]),
            "fo_f16_to_f32": (f32, [C.c_uint16]),
            "fo_f32_to_f16": (C.c_uint16, [f32]),
            "fo_f32_to_f16_array": (None, [vp, sz, vp]),
            "fo_f16_to_f32_array": (None, [vp, sz, vp]),
            "fo_f32_to_f16_f16c": (i32, [vp, sz, vp]),
            "fo_philox4x32_10": (None, [vp, vp, vp]),
            "fo_random_bits_fill": (None, [vp, sz, u64, u64, u32, u32]),
            "fo_normal_fill": (None, [vp, sz, u64, u32, f32, f32]),
            "fo_uniform_u32_fill": (None, [vp, sz, u64, u32, u32]),
            "fo_quantize_q8k": (None, [vp, sz, vp]),
            "fo_quantize_q8_0": (None, [vp, sz, vp]),
            "fo_quantize_q4k": (None, [vp, sz, vp]),
            "fo_quantize_q6k": (None, [vp, sz, vp]),
            "fo_quantize_rows": (None, [i32, vp, sz, sz, vp]),
            "fo_quantize_imatrix": (i32, [i32, vp, sz, vp, sz, vp]),
            "fo_dequantize": (None, [i32, vp, sz, vp]),
            "fo_q4k_unpack_scales": (None, [vp, vp, vp]),
            "fo_vec_dot_q4k_unopt": (f32, [sz, vp, vp]),
            "fo_vec_dot_q6k_unopt": (f32, [sz, vp, vp]),
            "fo_vec_dot_q8_0_unopt": (f32, [sz, vp, vp]),
            "fo_vec_dot_q4k_avx2": (f32, [sz, vp, vp]),
            "fo_vec_dot_q6k_avx2": (f32, [sz, vp, vp]),
            "fo_vec_dot_q8_0_avx2": (f32, [sz, vp, vp]),
            "fo_have_avx2": (i32, []),
            "fo_block_isums": (None, [i32, sz, vp, vp, vp, vp]),
            "fo_matmul": (i32, [i32, sz, sz, sz, vp, vp, vp, i32, i32]),
            "fo_qmatmul_bytes": (i32, [i32, sz, sz, sz, sz, vp, sz, vp, sz, vp, sz, i32, i32]),
            "fo_moe_route": (None, [vp, sz, sz, sz, vp, vp, vp, vp, vp]),
            "fo_moe_ffn": (i32, [i32, sz, sz, sz, sz, sz, vp, vp, vp, vp, vp, vp, vp, i32, i32]),
            "fo_rms_norm": (None, [vp, vp, sz, sz, f32, vp]),
            "fo_rope_tables": (None, [C.c_double, sz, sz, sz, vp, vp]),
            "fo_rope": (None, [vp, vp, vp, sz, sz, sz, vp]),
            "fo_attention_decode": (None, [vp, vp, vp, sz, sz, sz, sz, f32, vp]),
            "fo_argmax": (sz, [vp, sz]),
        }
        for name, (res, args) in sigs.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(C.c_void_p)


# ---- f16 -------------------------------------------------------------------

def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, np.uint16)
    lib().fo_f32_to_f16_array(_p(x), x.size, _p(y))
    return y


def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    y = np.empty(h.shape, np.float32)
    lib().fo_f16_to_f32_array(_p(h), h.size, _p(y))
    return y


def f32_to_f16_f16c(x: np.ndarray):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, np.uint16)
    rc = lib().fo_f32_to_f16_f16c(_p(x), x.size, _p(y))
    return None if rc else y


# ---- RNG -------------------------------------------------------------------

def philox4x32_10(ctr, key) -> np.ndarray:
    c = np.asarray(ctr, np.uint32).copy()
    k = np.asarray(key, np.uint32).copy()
    out = np.empty(4, np.uint32)
    lib().fo_philox4x32_10(_p(c), _p(k), _p(out))
    return out


def random_bits(n: int, start: int, seed: int, base: int, stream: int) -> np.ndarray:
    out = np.empty(n, np.uint32)
    lib().fo_random_bits_fill(_p(out), n, start, seed, base, stream)
    return out


def normal(shape, seed: int, stream: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(shape, np.float32)
    lib().fo_normal_fill(_p(out), out.size, seed, stream, mean, std)
    return out


def uniform_u32(n: int, seed: int, stream: int, bound: int) -> np.ndarray:
    out = np.empty(n, np.uint32)
    lib().fo_uniform_u32_fill(_p(out), n, seed, stream, bound)
    return out


# ---- quantize / dequantize ---------------------------------------------------

def quantize(dtype: int, x: np.ndarray) -> np.ndarray:
    """Row-wise from_float: x [..., k] f32 -> blocks [..., k/blk]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    k = x.shape[-1]
    bs = BLOCK_SIZE[dtype]
    assert k % bs == 0
    rows = x.size // k
    y = np.zeros(x.shape[:-1] + (k // bs,), BLOCK_DTYPE[dtype])
    lib().fo_quantize_rows(dtype, _p(x), rows, k, _p(y))
    return y


def quantize_imatrix(dtype: int, x: np.ndarray, imatrix: np.ndarray, n_per_row: int) -> np.ndarray:
    """from_float_imatrix (Q4_K / Q6_K) over the flattened x: superblock s uses
    the importance weights imatrix[(s % (n_per_row / 256)) * 256 ...]."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(imatrix, dtype=np.float32)
    assert w.size >= n_per_row and x.size % 256 == 0
    y = np.zeros(x.shape[:-1] + (x.shape[-1] // 256,), BLOCK_DTYPE[dtype])
    rc = lib().fo_quantize_imatrix(dtype, _p(x), x.size, _p(w), n_per_row, _p(y))
    if rc:
        raise ValueError(f"quantize_imatrix: dtype {dtype}, n_per_row {n_per_row}")
    return y


def dequantize(dtype: int, blocks: np.ndarray) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks)
    k = blocks.shape[-1] * BLOCK_SIZE[dtype]
    rows = blocks.size // blocks.shape[-1]
    y = np.empty(blocks.shape[:-1] + (k,), np.float32)
    flat_b = blocks.reshape(rows, -1)
    flat_y = y.reshape(rows, k)
    for r in range(rows):
        lib().fo_dequantize(dtype, _p(flat_b[r]), k, _p(flat_y[r]))
    return y


def q4k_unpack_scales(packed12: np.ndarray):
    p = np.ascontiguousarray(packed12, np.uint8)
    sc = np.empty(8, np.uint8)
    mn = np.empty(8, np.uint8)
    lib().fo_q4k_unpack_scales(_p(p), _p(sc), _p(mn))
    return sc, mn


# ---- dots -------------------------------------------------------------------

def vec_dot(dtype: int, w_row: np.ndarray, a_row: np.ndarray, avx2: bool = False) -> float:
    k = w_row.shape[-1] * BLOCK_SIZE[dtype]
    name = {Q4K: "q4k", Q6K: "q6k", Q8_0: "q8_0"}[dtype]
    fn = getattr(lib(), f"fo_vec_dot_{name}_{'avx2' if avx2 else 'unopt'}")
    return float(fn(k, _p(np.ascontiguousarray(w_row)), _p(np.ascontiguousarray(a_row))))


def block_isums(dtype: int, w: np.ndarray, a: np.ndarray):
    """Per-superblock integer sums for every (m, n, b): returns (isum, msum)
    of shape [m, n, k/blk] with w [n, kb] and a [m, kb]."""
    w = np.ascontiguousarray(w)
    a = np.ascontiguousarray(a)
    n, kb = w.shape
    m = a.shape[0]
    k = kb * BLOCK_SIZE[dtype]
    isum = np.zeros((m, n, kb), np.int32)
    msum = np.zeros((m, n, kb), np.int32)
    for i in range(m):
        for j in range(n):
            lib().fo_block_isums(dtype, k, _p(w[j]), _p(a[i]), _p(isum[i, j]), _p(msum[i, j]))
    return isum, msum


def have_avx2() -> bool:
    return bool(lib().fo_have_avx2())


def matmul(dtype: int, x: np.ndarray, w: np.ndarray, avx2: bool = True, threads: int = 0) -> np.ndarray:
    """fuel_quantized::matmul::<T>((m,k,n), x, w): x [m,k] f32, w [n, k/blk]."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w)
    m, k = x.shape
    n = w.shape[0]
    y = np.empty((m, n), np.float32)
    rc = lib().fo_matmul(dtype, m, k, n, _p(x), _p(w), _p(y), int(avx2 and have_avx2()), threads)
    if rc:
        raise ValueError(f"fo_matmul status {rc}")
    return y


def matmul_f16(dtype: int, x16: np.ndarray, w: np.ndarray, avx2: bool = True, threads: int = 0) -> np.ndarray:
    """fuel_quantized::matmul_f16::<T> (k_quants.rs:2333-2374): x [m,k] f16
    (as uint16 bits) widened to f32 (f16::to_f32), the f32 matmul, then each
    output rounded by f16::from_f32; returns uint16 bits [m, n]."""
    x32 = f16_bits_to_f32(np.ascontiguousarray(x16, np.uint16))
    return f32_to_f16_bits(matmul(dtype, x32, w, avx2, threads))


def moe_route(logits: np.ndarray, topk: int):
    logits = np.ascontiguousarray(logits, np.float32)
    t, e = logits.shape
    ids = np.empty((t, topk), np.int32)
    w = np.empty((t, topk), np.float32)
    off = np.empty(e + 1, np.int32)
    sorted_ids = np.empty(t * topk, np.int32)
    slot = np.empty(t * topk, np.int32)
    lib().fo_moe_route(_p(logits), t, e, topk, _p(ids), _p(w), _p(off), _p(sorted_ids), _p(slot))
    return ids, w, off, sorted_ids, slot


def moe_ffn(dtype, x, ids, w, w_gate, w_up, w_down, avx2=True, threads=0):
    x = np.ascontiguousarray(x, np.float32)
    t, d = x.shape
    topk = ids.shape[1]
    e = w_gate.shape[0]
    ffn = w_gate.shape[1]
    out = np.empty((t, d), np.float32)
    rc = lib().fo_moe_ffn(dtype, t, d, ffn, e, topk, _p(x), _p(np.ascontiguousarray(ids, np.int32)),
                          _p(np.ascontiguousarray(w, np.float32)), _p(np.ascontiguousarray(w_gate)),
                          _p(np.ascontiguousarray(w_up)), _p(np.ascontiguousarray(w_down)), _p(out),
                          int(avx2 and have_avx2()), threads)
    if rc:
        raise ValueError(f"fo_moe_ffn status {rc}")
    return out


# ---- LLaMA decoder pieces ----------------------------------------------------

def rms_norm(x: np.ndarray, gain: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    gain = np.ascontiguousarray(gain, np.float32)
    dim = x.shape[-1]
    y = np.empty_like(x)
    lib().fo_rms_norm(_p(x), _p(gain), x.size // dim, dim, eps, _p(y))
    return y


def rope_tables(base: float, start_pos: int, seq: int, head_dim: int):
    c = np.empty((seq, head_dim), np.float32)
    s = np.empty((seq, head_dim), np.float32)
    lib().fo_rope_tables(base, start_pos, seq, head_dim, _p(c), _p(s))
    return c, s


def rope(x: np.ndarray, cos_t: np.ndarray, sin_t: np.ndarray) -> np.ndarray:
    """x [..., seq, head_dim] with tables [seq, head_dim]."""
    x = np.ascontiguousarray(x, np.float32)
    seq, hd = x.shape[-2:]
    y = np.empty_like(x)
    lib().fo_rope(_p(x), _p(np.ascontiguousarray(cos_t, np.float32)), _p(np.ascontiguousarray(sin_t, np.float32)),
                  x.size // (seq * hd), seq, hd, _p(y))
    return y


def attention_decode(q: np.ndarray, k: np.ndarray, v: np.ndarray, n_ctx: int, scale: float) -> np.ndarray:
    """q [heads, hd]; k, v [heads, stride, hd] (first n_ctx rows used)."""
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    heads, stride, hd = k.shape
    out = np.empty((heads, hd), np.float32)
    lib().fo_attention_decode(_p(q), _p(k), _p(v), heads, n_ctx, stride, hd, scale, _p(out))
    return out


def argmax(x: np.ndarray) -> int:
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    return int(lib().fo_argmax(_p(x), x.size))
