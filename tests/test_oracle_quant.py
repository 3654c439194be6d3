"""Pins of the oracle's quantizers and dequantizers (CPU only).

Activation quantizers (BlockQ8K::from_float k_quants.rs:2230-2267,
BlockQ8_0::from_float :629-658) are pinned by closed forms on integer inputs,
the first-index tie rule with planted duplicates, the all-zero branch and the
rounding / range invariants.  Weight formats are pinned by crafted blocks with
known values (to_float), the two scale-unpack routines agreeing on random
bytes, the all-ones Q6K case of fuel-dispatch/src/pipelined.rs:10073-10139
worked out by hand, and from_float -> to_float error bounds.

The exact bytes of BlockQ4K::from_float / BlockQ6K::from_float are pinned
by the hand-derived known-answer blocks of test_oracle_quant_kat.py.
"""
import numpy as np

import oracle as O
from blockref import q4k_fields, q6k_fields


def q8k(x):
    return O.quantize(O.Q8K, np.asarray(x, np.float32).reshape(1, -1))[0]


def test_q8k_integer_closed_form():
    # x = j - 128: the first |x| max is x[0] = -128, so iscale = 1 and q = x.
    x = np.arange(256, dtype=np.float32) - 128
    b = q8k(x)[0]
    assert b["d"] == 1.0
    assert np.array_equal(b["qs"].astype(np.int64), x.astype(np.int64))
    assert np.array_equal(b["bsums"], x.reshape(16, 16).sum(1).astype(np.int16))


def test_q8k_first_index_tie_rule():
    x = np.zeros(256, np.float32)
    x[3], x[10] = -5.0, 5.0      # equal |x|: the earlier (-5) sets the sign
    b = q8k(x)[0]
    assert b["qs"][3] == -128 and b["qs"][10] == 127   # +128 saturates at 127
    assert b["d"] == np.float32(1.0) / (np.float32(-128.0) / np.float32(-5.0))
    x[3], x[10] = 5.0, -5.0
    b = q8k(x)[0]
    assert b["qs"][3] == -128 and b["qs"][10] == 127
    assert b["d"] < 0


def test_q8k_zero_block():
    b = q8k(np.zeros(512, np.float32))
    assert np.all(b["d"] == 0) and np.all(b["qs"] == 0) and np.all(b["bsums"] == 0)


def test_q8k_invariants_random():
    x = O.normal((8, 1024), seed=5, stream=11)
    blocks = O.quantize(O.Q8K, x)
    xb = x.reshape(8, 4, 256)
    qs = blocks["qs"].astype(np.int64)
    d = blocks["d"].astype(np.float64)
    assert np.array_equal(blocks["bsums"].astype(np.int64), qs.reshape(8, 4, 16, 16).sum(-1))
    # the element with the first max |x| maps to exactly -128
    imax = np.abs(xb).argmax(-1)
    assert np.all(np.take_along_axis(qs, imax[..., None], -1) == -128)
    # |x - d*q| <= |d|/2 (q = round(x/d) with d = -max/128), except at the +127 clip
    err = np.abs(xb - d[..., None] * qs)
    clip = qs == 127
    assert np.all(err[~clip] <= np.abs(d)[..., None].repeat(256, -1)[~clip] * 0.5000001)


def test_q8_0_invariants_random():
    x = O.normal((4, 4096), seed=6, stream=12)
    blocks = O.quantize(O.Q8_0, x)
    xb = x.reshape(4, 128, 32).astype(np.float32)
    amax = np.abs(xb).max(-1)
    d = (amax / np.float32(127)).astype(np.float32)
    assert np.array_equal(blocks["d"], d.astype(np.float16).view(np.uint16))
    qs = blocks["qs"].astype(np.int64)
    assert np.all(np.abs(qs) <= 127)
    idx = np.abs(xb).argmax(-1)
    assert np.all(np.abs(np.take_along_axis(qs, idx[..., None], -1)) == 127)
    idv = (np.float32(1) / d).astype(np.float32)
    assert np.all(np.abs(xb * idv[..., None] - qs) <= 0.5)


def test_q4k_crafted_block_to_float():
    b = np.zeros(1, O.BLOCK_Q4K)
    b["d"] = np.float16(0.5).view(np.uint16)
    b["dmin"] = np.float16(0.25).view(np.uint16)
    sc = np.array([1, 2, 3, 4, 33, 40, 50, 63])
    mn = np.array([0, 5, 10, 15, 20, 25, 48, 62])
    s = np.zeros(12, np.int64)
    for j in range(8):   # inverse of get_scale_min_k4 (utils.rs:50-60)
        if j < 4:
            s[j] |= sc[j]
            s[j + 4] |= mn[j]
        else:
            s[j + 4] |= (sc[j] & 0xF) | ((mn[j] & 0xF) << 4)
            s[j - 4] |= (sc[j] >> 4) << 6
            s[j] |= (mn[j] >> 4) << 6
    b["scales"] = s.astype(np.uint8)
    q = (np.arange(256) * 7) % 16
    qs = np.zeros(128, np.int64)
    for c in range(4):
        qs[32 * c:32 * c + 32] = q[64 * c:64 * c + 32] | (q[64 * c + 32:64 * c + 64] << 4)
    b["qs"] = qs.astype(np.uint8)
    y = O.dequantize(O.Q4K, b)
    sub = np.arange(256) // 32
    want = np.float32(0.5) * sc[sub].astype(np.float32) * q.astype(np.float32) - \
        np.float32(0.25) * mn[sub].astype(np.float32)
    assert np.array_equal(y, want.astype(np.float32))
    # both scale unpack routes of the reference agree with the format
    sc8, mn8 = O.q4k_unpack_scales(b["scales"][0])
    assert np.array_equal(sc8, sc) and np.array_equal(mn8, mn)


def test_q4k_scale_unpack_routes_agree_random_bytes():
    rng = np.random.default_rng(0)
    for _ in range(200):
        raw = rng.integers(0, 256, 12).astype(np.uint8)
        sc8, mn8 = O.q4k_unpack_scales(raw)
        blk = np.zeros(1, O.BLOCK_Q4K)
        blk["scales"] = raw
        _, _, sc, mn, _ = q4k_fields(blk)
        assert np.array_equal(sc8, sc[0]) and np.array_equal(mn8, mn[0])


def test_q6k_all_ones_known_answer():
    # pipelined.rs:10073-10139 quantizes an all-ones [2, 256] weight.  By hand
    # (utils.rs:62-226 with rmse_type 1): every group scale is -1/32, so
    # max_scale = -1/32, iscale = 4096, d = f16(2^-12), scales = -128 and every
    # code is L = 0 (value (0 - 32) * 2^-12 * -128 = 1).
    b = O.quantize(O.Q6K, np.ones((2, 256), np.float32))
    assert np.all(b["d"] == 0x0C00)
    assert np.all(b["scales"] == -128)
    assert np.all(b["ql"] == 0) and np.all(b["qh"] == 0)
    assert np.all(O.dequantize(O.Q6K, b) == 1.0)


def test_q6k_crafted_block_to_float():
    rng = np.random.default_rng(1)
    b = np.zeros(1, O.BLOCK_Q6K)
    b["ql"] = rng.integers(0, 256, 128).astype(np.uint8)
    b["qh"] = rng.integers(0, 256, 64).astype(np.uint8)
    b["scales"] = rng.integers(-128, 128, 16).astype(np.int8)
    b["d"] = np.float16(0.125).view(np.uint16)
    d, sc, q = q6k_fields(b)
    want = (np.float32(0.125) * sc[0][np.arange(256) // 16].astype(np.float32)) * q[0].astype(np.float32)
    assert np.array_equal(O.dequantize(O.Q6K, b), want.astype(np.float32))


def test_weight_quantizers_error_bounds():
    w = O.normal((16, 2048), seed=3, stream=4, std=0.02)
    for dt, tol in ((O.Q4K, 0.13), (O.Q6K, 0.035), (O.Q8_0, 0.008)):
        blocks = O.quantize(dt, w)
        back = O.dequantize(dt, blocks)
        bs = O.BLOCK_SIZE[dt]
        span = np.ptp(w.reshape(16, -1, bs), axis=-1)[..., None]
        rel = np.abs(back - w).reshape(16, -1, bs) / span
        assert rel.max() < tol, (dt, rel.max())
    q4 = O.quantize(O.Q4K, w)
    _, _, sc, mn, q = q4k_fields(q4)
    assert sc.max() <= 63 and mn.max() <= 63 and q.max() <= 15
    # every 6-bit scale range is used: the largest sub-block scale maps to 63
    assert np.all(sc.max(-1) == 63)
