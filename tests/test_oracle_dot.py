"""Pins of the oracle's block dot products and matmul<T> (CPU only).

* Integer stage (isum / msum of vec_dot, k_quants.rs:1388-1468, 1946-2003,
  674-692): equal to brute-force element sums from the format decoders in
  tests/blockref.py.
* f32 stage: vec_dot_unopt and the AVX2 vec_dot (avx.rs) agree with the exact
  float64 value of sum_b d_w*d_a*isum - dmin_w*d_a*msum, and with a float64
  GEMV over to_float(W) and to_float(Q8(x)) (a dropped min term or a wrong
  sign fails this by orders of magnitude).
* matmul<T> (k_quants.rs:2284-2331): the unit-weight closed form of
  fuel-cpu-backend/src/byte_kernels.rs:9718-9750 restated for Q4K, zero
  activations, and qmatmul_generic_f32's validation (byte_kernels.rs:4767-4806).
"""
import numpy as np
import pytest

import oracle as O
from blockref import brute_isums, exact_dot64, rel_err

DTYPES = [O.Q4K, O.Q6K, O.Q8_0]


def _case(dt, m=3, n=24, k=1024, seed=0):
    x = O.normal((m, k), seed=seed, stream=1)
    w = O.normal((n, k), seed=seed, stream=2, std=0.02)
    wq = O.quantize(dt, w)
    aq = O.quantize(O.VEC_DOT_TYPE[dt], x)
    return x, w, wq, aq


@pytest.mark.parametrize("dt", DTYPES)
def test_block_isums_match_brute_force(dt):
    _, _, wq, aq = _case(dt)
    isum, msum = O.block_isums(dt, wq, aq)
    bi, bm = brute_isums(dt, wq, aq)
    assert np.array_equal(isum, bi)
    assert np.array_equal(msum, bm)


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("avx2", [False, True])
def test_vec_dot_matches_exact_value(dt, avx2):
    if avx2 and not O.have_avx2():
        pytest.skip("host lacks AVX2")
    x, w, wq, aq = _case(dt)
    exact = exact_dot64(dt, wq, aq)
    got = np.array([[O.vec_dot(dt, wq[j], aq[i], avx2=avx2) for j in range(wq.shape[0])]
                    for i in range(aq.shape[0])])
    assert rel_err(got, exact) < 1e-6
    # and against a float64 GEMV over the dequantized operands
    wd = O.dequantize(dt, wq).astype(np.float64)
    ad = O.dequantize(O.VEC_DOT_TYPE[dt], aq).astype(np.float64)
    assert rel_err(got, ad @ wd.T) < 1e-5
    # quantization keeps the product close to the float GEMV (sanity)
    assert rel_err(got, x.astype(np.float64) @ w.T.astype(np.float64)) < 6e-2


@pytest.mark.parametrize("dt", DTYPES)
def test_matmul_threads_and_paths_agree(dt):
    x, _, wq, aq = _case(dt, m=2, n=300, k=512)
    y1 = O.matmul(dt, x, wq, avx2=False, threads=1)
    y4 = O.matmul(dt, x, wq, avx2=False, threads=4)
    assert np.array_equal(y1, y4)   # the column split does not change arithmetic
    if O.have_avx2():
        ya = O.matmul(dt, x, wq, avx2=True)
        assert rel_err(ya, y1) < 1e-6


def test_matmul_q4k_unit_weight_sums_activations():
    # byte_kernels.rs:9718-9750 pattern: every weight equal to 1 so A @ W^T is the
    # row sum.  Q4K: d = 1, dmin = 0, all 6-bit scales 1, every nibble 1.
    n, k = 2, 512
    b = np.zeros((n, k // 256), O.BLOCK_Q4K)
    b["d"] = np.float16(1.0).view(np.uint16)
    b["scales"] = np.array([1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1], np.uint8)
    b["qs"] = 0x11
    assert np.all(O.dequantize(O.Q4K, b) == 1.0)
    x = (np.arange(1, k + 1, dtype=np.float32) / 100.0).reshape(1, k)
    a = O.quantize(O.Q8K, x)[0]
    exact = float((a["d"].astype(np.float64) * a["qs"].astype(np.int64).sum(-1)).sum())
    bound = float((np.abs(a["d"].astype(np.float64)) * 256 / 2).sum())
    for avx2 in (False, True):
        y = O.matmul(O.Q4K, x, b, avx2=avx2)
        assert np.all(np.abs(y - exact) <= 1e-6 * abs(exact)), (y, exact)
        assert np.all(np.abs(y - x.sum(dtype=np.float64)) <= bound)


def test_matmul_zero_activations():
    _, _, wq, _ = _case(O.Q6K, n=4, k=256)
    assert np.all(O.matmul(O.Q6K, np.zeros((1, 256), np.float32), wq) == 0.0)


def test_qmatmul_bytes_validation():
    import ctypes as C
    L = O.lib()
    act = np.zeros(33, np.float32)
    w = np.zeros(34, np.uint8)
    out = np.zeros(1, np.float32)
    p = lambda a: a.ctypes.data_as(C.c_void_p)
    # k = 33 is not a multiple of 32
    assert L.fo_qmatmul_bytes(O.Q8_0, 1, 1, 1, 33, p(act), 132, p(w), 34, p(out), 4, 0, 1) == 2
    # weight byte mismatch
    act = np.zeros(32, np.float32)
    assert L.fo_qmatmul_bytes(O.Q8_0, 1, 1, 1, 32, p(act), 128, p(w), 33, p(out), 4, 0, 1) == 2
    # zero rows is a no-op
    assert L.fo_qmatmul_bytes(O.Q8_0, 1, 0, 1, 32, p(act), 0, p(w), 34, p(out), 0, 0, 1) == 0
