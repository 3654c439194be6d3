"""The oracle's from_float_imatrix (quantize_imatrix on the trait seam):
BlockQ4K k_quants.rs:1530-1593 with make_qkx3_quants (utils.rs:358-469) and
make_qp_quants (utils.rs:472-563); BlockQ6K k_quants.rs:2077-2145 with
make_qx_quants (utils.rs:62-226) weighted by the importance matrix.

What pins them:

* Q6K reduces to from_float: with importance weights w = x*x, make_qx_quants
  with qw = w computes exactly what from_float's rmse_type-1 weights (x*x)
  compute, and the rest of the two functions is the same code; so
  quantize_imatrix(x, x*x) must give from_float's bytes, which the hand-derived
  known-answer blocks of weight_kat pin.
* Q4K known answers worked out by hand: sub-blocks on an exact 16-level grid
  make every make_qkx3_quants candidate fit with zero weighted error at the
  first pass, so it returns (s, -min) exactly whatever the weights are, and
  make_qp_quants over equal (or zero) sub-block scales lands on 63 (or 0) codes
  and scale ~ s/63; the f16 d / dmin, the 6-bit packing and the codes follow.
* The weighting itself: the importance weight of element l of sub-block j is
  imatrix[32 j + l] (a heavy weight there fits that element much more
  closely), weights scale linearly with the importance matrix (doubling it
  leaves every byte unchanged: every sum doubles exactly), and
  sqrt(sigma2 + x^2) is homogeneous in x (doubling x doubles d and dmin and
  keeps every scale and code), and column blocks repeat per n_per_row.
* The importance formula itself (sigma2 = 2 sum(x^2) / 256 and the square
  root in w = imatrix * sqrt(sigma2 + x^2), k_quants.rs:1539-1548): a block
  whose dmin is a weighted least-squares fit over the sub-block weights sw_j,
  worked out in float64 with its rounding margins (weight_kat); dropping the
  factor 2 or the square root moves dmin's f16 bits, and copies of the oracle
  with either slip planted fail it.
"""
import os

import numpy as np
import pytest

import oracle as O
from weight_kat import CASES, _q4k_block

S = np.float32(2.0 ** -6)


def d_of(v):
    """f16 bits of the value nearest v (float64): d = f16(s / 63) etc."""
    return int(np.float16(v).view(np.uint16))


@pytest.mark.parametrize("name", sorted(n for n in CASES if CASES[n][0] == O.Q6K))
def test_q6k_imatrix_with_x_squared_is_from_float(name):
    _, case = CASES[name]
    x, want = case()
    got = O.quantize_imatrix(O.Q6K, x.reshape(1, 256), (x * x).astype(np.float32), 256)
    assert got.tobytes() == want.tobytes(), name


def test_q6k_imatrix_with_x_squared_is_from_float_random_rows():
    x = O.normal((5, 768), seed=11, stream=3)
    for r in range(5):
        got = O.quantize_imatrix(O.Q6K, x[r:r + 1], (x[r] * x[r]).astype(np.float32), 768)
        assert got.tobytes() == O.quantize(O.Q6K, x[r:r + 1]).tobytes()


def _grid(j, shift=0):
    return np.array([(l + shift * j) % 16 for l in range(32)], np.int64)


def _weights(seed):
    return np.random.default_rng(seed).uniform(0.05, 3.0, 256).astype(np.float32)


@pytest.mark.parametrize("seed", [0, 1])
def test_q4k_imatrix_grid_known_answer(seed):
    """Eight grid sub-blocks x = k * S (k in 0..15, both ends present): each
    make_qkx3_quants returns (S, -0.0); make_qp_quants of eight S gives codes 63
    and ~S/63; the mins are all zero (dmin 0, codes 0).  Expected bytes: d =
    f16(S/63), dmin 0, ls = 63 / lm = 0 packed, codes k."""
    codes = np.stack([_grid(j, 1) for j in range(8)])
    x = (codes.reshape(256) * S).astype(np.float32)
    want = _q4k_block(d_of(float(S) / 63), 0, [63] * 8, [0] * 8, codes.reshape(256))
    got = O.quantize_imatrix(O.Q4K, x.reshape(1, 256), _weights(seed), 256)
    assert got.tobytes() == want.tobytes()


@pytest.mark.parametrize("seed", [2, 3])
def test_q4k_imatrix_grid_with_min_known_answer(seed):
    """x = -4S + k * S: the grid from min -4S; (S, 4S) per sub-block, so
    make_qp_quants gives d ~ S/63 and dmin ~ 4S/63 = 4 d exactly after f16,
    every 6-bit scale and min 63 (all twelve packed bytes 255), codes k."""
    codes = np.stack([_grid(j, 3) for j in range(8)])
    x = ((codes.reshape(256) - 4) * S).astype(np.float32)
    dbits = d_of(float(S) / 63)
    want = _q4k_block(dbits, d_of(4 * float(S) / 63), [63] * 8, [63] * 8, codes.reshape(256))
    assert bytes(want["scales"][0]) == b"\xff" * 12
    got = O.quantize_imatrix(O.Q4K, x.reshape(1, 256), _weights(seed), 256)
    assert got.tobytes() == want.tobytes()


def test_q4k_imatrix_zero_subblocks_known_answer():
    """Even sub-blocks on the grid, odd ones all zero: the zero sub-blocks give
    (0, -0.0), so the scale codes are 63, 0, 63, 0, ... (the descent keeps a
    zero value at code 0), d ~ S/63, dmin 0; zero sub-blocks keep codes 0."""
    codes = np.stack([_grid(j, 5) if j % 2 == 0 else np.zeros(32, np.int64) for j in range(8)])
    x = (codes.reshape(256) * S).astype(np.float32)
    ls = [63 if j % 2 == 0 else 0 for j in range(8)]
    want = _q4k_block(d_of(float(S) / 63), 0, ls, [0] * 8, codes.reshape(256))
    got = O.quantize_imatrix(O.Q4K, x.reshape(1, 256), _weights(4), 256)
    assert got.tobytes() == want.tobytes()
    assert list(want["scales"][0]) == [255, 0, 255, 0, 0, 0, 0, 0, 15, 0, 15, 0]


def test_q4k_imatrix_weights_are_linear_in_the_importance_matrix():
    x = O.normal((4, 512), seed=21, stream=1)
    w = _weights(7)[np.arange(512) % 256] * np.float32(0.5)
    a = O.quantize_imatrix(O.Q4K, x, w, 512)
    b = O.quantize_imatrix(O.Q4K, x, (w * 2).astype(np.float32), 512)
    assert a.tobytes() == b.tobytes()


def test_q4k_imatrix_weights_are_homogeneous_in_x():
    """Doubling x doubles sqrt(sigma2 + x^2) and every scale and min: d and
    dmin double (f16 exponent + 1), the packed scales and the codes stay."""
    x = O.normal((4, 512), seed=22, stream=1)
    w = np.random.default_rng(8).uniform(0.1, 2.0, 512).astype(np.float32)
    a = O.quantize_imatrix(O.Q4K, x, w, 512)
    b = O.quantize_imatrix(O.Q4K, (x * 2).astype(np.float32), w, 512)
    assert np.array_equal(a["scales"], b["scales"]) and np.array_equal(a["qs"], b["qs"])
    da, db = O.f16_bits_to_f32(a["d"]), O.f16_bits_to_f32(b["d"])
    ma, mb = O.f16_bits_to_f32(a["dmin"]), O.f16_bits_to_f32(b["dmin"])
    assert np.array_equal(db, 2 * da) and np.array_equal(mb, 2 * ma)


def test_q4k_imatrix_weight_index():
    """Element l of sub-block j takes importance imatrix[32 j + l]: weighting
    one element 1e4 times its neighbours fits it far more closely than
    weighting the element 7 places away (its mean reconstruction error drops
    well below the other choice's)."""
    x = O.normal((64, 256), seed=23, stream=1)
    err_here, err_there = [], []
    for j, l in [(1, 5), (4, 30), (6, 17)]:
        p = 32 * j + l
        for target, out in ((p, err_here), ((p + 7) % 256, err_there)):
            w = np.full(256, 1e-4, np.float32)
            w[target] = 1.0
            y = O.dequantize(O.Q4K, O.quantize_imatrix(O.Q4K, x, w, 256))
            out.append(np.abs(y[:, p] - x[:, p]).mean())
    assert np.mean(err_here) < 0.5 * np.mean(err_there), (err_here, err_there)


def test_imatrix_column_blocks_repeat_per_row():
    """Superblock s uses column block s % (n_per_row / 256): rows of a matrix
    share the importance matrix; with n_per_row = 256 every superblock uses the
    first 256 weights."""
    x = O.normal((3, 768), seed=24, stream=1)
    w = np.random.default_rng(9).uniform(0.1, 2.0, 768).astype(np.float32)
    for dt in (O.Q4K, O.Q6K):
        whole = O.quantize_imatrix(dt, x, w, 768)
        for r in range(3):
            assert whole[r].tobytes() == O.quantize_imatrix(dt, x[r:r + 1], w, 768).tobytes()
        tiled = O.quantize_imatrix(dt, x, w, 256)
        again = O.quantize_imatrix(dt, x, np.tile(w[:256], 3), 768)
        assert tiled.tobytes() == again.tobytes()


def test_imatrix_types_and_row_sizes():
    x = O.normal((1, 256), seed=25, stream=1)
    w = np.ones(256, np.float32)
    with pytest.raises(ValueError):
        O.quantize_imatrix(O.Q8_0, x, w, 256)
    with pytest.raises(ValueError):
        O.quantize_imatrix(O.Q4K, x, w, 100)


def test_q4k_imatrix_importance_formula_known_answer():
    """The block of weight_kat.q4k_imatrix_formula_case: its dmin is the
    weighted least-squares fit over sw_j = sum imatrix * sqrt(sigma2 + x^2),
    sigma2 = 2 sum(x^2) / 256, worked out in float64; the margins show that
    neither the f16 rounding of dmin nor a code of the search sits near a
    boundary."""
    from weight_kat import code_margin, imatrix_margins, q4k_imatrix_formula_case

    x, qw, want = q4k_imatrix_formula_case()
    f16_margin, descent_margin = imatrix_margins(x, qw)
    assert f16_margin > 0.3 and descent_margin > 0.15, (f16_margin, descent_margin)
    assert code_margin(O.Q4K, x, want) < 0.1
    got = O.quantize_imatrix(O.Q4K, x.reshape(1, 256), qw, 256)
    assert got.tobytes() == want.tobytes(), (got, want)


def test_q4k_imatrix_formula_slips_change_the_known_answer():
    """Each plausible slip of the importance formula moves dmin's f16 bits in
    the closed form, by more than one unit."""
    from weight_kat import imatrix_formula_dmin, imatrix_formula_inputs

    x, qw = imatrix_formula_inputs()
    bits = lambda v: int(np.float16(v).view(np.uint16))
    right = bits(imatrix_formula_dmin(x, qw))
    for slip in ({"sigma2_factor": 1.0}, {"sqrt": False}, {"sigma2_factor": 1.0, "sqrt": False}):
        assert abs(bits(imatrix_formula_dmin(x, qw, **slip)) - right) >= 2, slip


MUTATIONS = {
    "sigma2 without the factor 2": ("float sigma2 = 2.0f * sum_x2 / (float)FO_QK_K;",
                                    "float sigma2 = sum_x2 / (float)FO_QK_K;"),
    "weights without the square root": ("weights[l] = qw[32 * j + l] * sqrtf(sigma2 + xe * xe);",
                                        "weights[l] = qw[32 * j + l] * (sigma2 + xe * xe);"),
}


@pytest.mark.parametrize("name", [None] + sorted(MUTATIONS))
def test_q4k_imatrix_known_answer_catches_a_planted_slip(tmp_path, name):
    """The known answer fails a copy of the oracle with the slip planted in its
    Q4K from_float_imatrix (built here with the oracle's own flags), and passes
    the unmodified copy built the same way."""
    import ctypes
    import shutil
    import subprocess

    from weight_kat import q4k_imatrix_formula_case

    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    src = open(os.path.join(os.path.dirname(O.__file__), "fuel_oracle.c")).read()
    if name is not None:
        old, new = MUTATIONS[name]
        assert src.count(old) == 1, f"the line to mutate is not in the oracle: {old}"
        src = src.replace(old, new)
    d = tmp_path / "mut"
    d.mkdir()
    shutil.copy(os.path.join(os.path.dirname(O.__file__), "fuel_oracle.h"), d / "fuel_oracle.h")
    (d / "fuel_oracle.c").write_text(src)
    so = d / "libmut.so"
    subprocess.run([cc, "-O2", "-std=c11", "-fPIC", "-fopenmp", "-ffp-contract=off", "-fno-fast-math", "-shared",
                    "-o", str(so), str(d / "fuel_oracle.c"), "-lm"], check=True)
    lib = ctypes.CDLL(str(so))
    lib.fo_quantize_imatrix.restype = ctypes.c_int
    lib.fo_quantize_imatrix.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p,
                                        ctypes.c_size_t, ctypes.c_void_p]
    x, qw, want = q4k_imatrix_formula_case()
    got = np.zeros(1, O.BLOCK_Q4K)
    assert lib.fo_quantize_imatrix(O.Q4K, x.ctypes.data, 256, qw.ctypes.data, 256, got.ctypes.data) == 0
    if name is None:
        assert got.tobytes() == want.tobytes()
    else:
        assert got.tobytes() != want.tobytes(), name
