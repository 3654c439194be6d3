"""Pins of the oracle's Philox generator and f16 conversions (CPU only).

Philox-4x32-10 is checked against the 55 Random123 known-answer vectors that
fuel's own tests hold (fuel-cpu-kernels/src/philox_kat.rs), extracted into
tests/golden/philox4x32_10_kat.json by tests/golden/make_philox_kat.py.
f16 -> f32 is checked exhaustively (all 65,536 patterns), the reference's own
strategy (fuel-graph/src/registry/qmatmul.rs:363-378), against numpy's IEEE
conversion; f32 -> f16 (half::f16::from_f32, round-to-nearest-even) against
numpy and the F16C instruction over a strided sweep of all f32 patterns.
"""
import json
import os

import numpy as np
import pytest

import oracle as O

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "philox4x32_10_kat.json")


def test_philox_random123_kat():
    vecs = json.load(open(GOLDEN))["vectors"]
    assert len(vecs) == 55
    for v in vecs:
        got = O.philox4x32_10(v["ctr"], v["key"])
        assert got.tolist() == v["out"], v


def test_random_bits_counter_mapping():
    # philox.rs:91-133: element i is lane i%4 of the block at counter
    # [i/4 lo, i/4 hi, base, stream] with key = seed split little-endian.
    seed, base, stream = 0x1234_5678_9ABC_DEF0, 7, 3
    bits = O.random_bits(37, 0, seed, base, stream)
    key = [seed & 0xFFFFFFFF, seed >> 32]
    for i in range(37):
        blk = O.philox4x32_10([i // 4, 0, base, stream], key)
        assert bits[i] == blk[i % 4]
    # a fill that starts mid-block continues the same global sequence
    tail = O.random_bits(30, 7, seed, base, stream)
    assert np.array_equal(tail, bits[7:37])


def test_normal_generator_moments_and_determinism():
    a = O.normal((1 << 20,), seed=9, stream=1)
    b = O.normal((1 << 20,), seed=9, stream=1)
    c = O.normal((1 << 20,), seed=9, stream=2)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    assert abs(a.mean()) < 5e-3 and abs(a.std() - 1.0) < 5e-3
    w = O.normal((1 << 18,), seed=9, stream=1, std=0.02)
    assert abs(w.std() - 0.02) < 2e-4


def test_f16_to_f32_exhaustive():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = O.f16_bits_to_f32(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def _f32_sweep(stride: int) -> np.ndarray:
    bits = np.arange(0, 1 << 32, stride, dtype=np.uint64).astype(np.uint32)
    # every f16 rounding boundary region: halfway points and their neighbours
    h = np.arange(0, 0x7C00, dtype=np.uint32)
    f = h.astype(np.uint16).view(np.float16).astype(np.float32).view(np.uint32)
    mids = (f[:-1].astype(np.uint64) + f[1:].astype(np.uint64)) // 2
    edge = np.concatenate([mids - 1, mids, mids + 1]).astype(np.uint32)
    edge = np.concatenate([edge, edge | np.uint32(0x80000000)])
    return np.concatenate([bits, edge]).view(np.float32)


def test_f32_to_f16_rne_sweep():
    x = _f32_sweep(stride=4099)
    got = O.f32_to_f16_bits(x)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], want[~nan])
    # NaN stays NaN (exponent all ones, non-zero mantissa)
    assert np.all((got[nan] & 0x7C00) == 0x7C00) and np.all((got[nan] & 0x3FF) != 0)


def test_f32_to_f16_matches_f16c():
    x = _f32_sweep(stride=65537)
    hw = O.f32_to_f16_f16c(x)
    if hw is None:
        pytest.skip("host lacks F16C")
    got = O.f32_to_f16_bits(x)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], hw[~nan])
