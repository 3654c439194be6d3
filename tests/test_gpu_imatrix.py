"""GPU parity of quantize_imatrix (frq_qstorage_quantize_imatrix, the trait
seam's quantize_imatrix / quantize_imatrix_onto) against the oracle's
from_float_imatrix (k_quants.rs:1530-1593 Q4_K, 2077-2145 Q6_K), byte for
byte, through the C ABI."""
import numpy as np
import pytest

import fuel_amd as F
import oracle as O
from fuel_amd._native import FRQ_INVALID, FRQ_UNSUPPORTED

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def device_imatrix(dev, dt, x, w, n_per_row):
    q = dev.qzeros(x.size, dt)
    q.quantize_imatrix(dev.from_numpy(x), w, n_per_row)
    return q.data()


@pytest.mark.parametrize("dt", [O.Q4K, O.Q6K])
@pytest.mark.parametrize("rows,k,npr", [(48, 2048, 2048), (7, 768, 768), (5, 1024, 256), (1, 4096, 4096)])
def test_device_quantize_imatrix_bit_exact(dev, dt, rows, k, npr):
    say("device from_float_imatrix", dt, rows, k, npr)
    x = np.concatenate([O.normal((rows - 1, k), seed=31 + k, stream=5, std=0.02),
                        O.normal((1, k), seed=32, stream=6, std=3.0)]) if rows > 1 else \
        O.normal((1, k), seed=33, stream=5)
    w = np.random.default_rng(k + npr).uniform(0.01, 4.0, npr).astype(np.float32)
    want = O.quantize_imatrix(dt, x, w, npr)
    got = device_imatrix(dev, dt, x, w, npr)
    if got != want.tobytes():
        g = np.frombuffer(got, O.BLOCK_DTYPE[dt]).reshape(want.shape)
        bad = np.nonzero(g.view(np.uint8).reshape(g.size, -1) != want.view(np.uint8).reshape(want.size, -1))
        pytest.fail(f"first differing blocks {np.unique(bad[0])[:8]}")


def test_device_quantize_imatrix_known_answers(dev):
    """Hand-derived blocks: Q6K with importance x*x gives from_float's known
    answers (weight_kat); Q4K grid sub-blocks give d = f16(S/63) and the 63
    codes whatever the importance weights."""
    from test_oracle_imatrix import S, _grid, _weights, d_of
    from weight_kat import CASES, _q4k_block

    names = [n for n in sorted(CASES) if CASES[n][0] == O.Q6K]
    xs, ws = zip(*(CASES[n][1]() for n in names))
    x = np.concatenate(xs)[None]
    for i, n in enumerate(names):
        xi = xs[i].reshape(1, 256)
        assert device_imatrix(dev, O.Q6K, xi, (xi * xi).astype(np.float32).reshape(256), 256) == ws[i].tobytes(), n
    codes = np.stack([_grid(j, 1) for j in range(8)]).reshape(256)
    xq = (codes * S).astype(np.float32).reshape(1, 256)
    want = _q4k_block(d_of(float(S) / 63), 0, [63] * 8, [0] * 8, codes)
    assert device_imatrix(dev, O.Q4K, xq, _weights(0), 256) == want.tobytes()


def test_device_quantize_imatrix_errors(dev):
    x = dev.from_numpy(O.normal((1, 512), seed=1, stream=1))
    w = np.ones(512, np.float32)
    q8 = dev.qzeros(512, O.Q8_0)
    with pytest.raises(F.FuelRocmError) as e:
        q8.quantize_imatrix(x, w, 512)
    assert e.value.status == FRQ_UNSUPPORTED
    q4 = dev.qzeros(512, O.Q4K)
    for bad in (0, 100, 300):
        with pytest.raises(F.FuelRocmError) as e:
            q4.quantize_imatrix(x, w, bad)
        assert e.value.status == FRQ_INVALID
    with pytest.raises(F.FuelRocmError):  # source size mismatch
        q4.quantize_imatrix(dev.from_numpy(O.normal((1, 256), seed=1, stream=1)), w, 256)


def test_device_quantize_imatrix_importance_formula(dev):
    """The importance-formula known answer (weight_kat.q4k_imatrix_formula_case:
    dmin is the float64 least-squares fit over sw_j = sum imatrix *
    sqrt(2 sum(x^2)/256 + x^2)) through frq_qstorage_quantize_imatrix."""
    from weight_kat import q4k_imatrix_formula_case

    x, qw, want = q4k_imatrix_formula_case()
    say("device from_float_imatrix, importance-formula block")
    assert device_imatrix(dev, O.Q4K, x.reshape(1, 256), qw, 256) == want.tobytes()
    # the same block repeated over a 4-superblock row, the importance matrix tiled per row
    x4 = np.tile(x, 4).reshape(1, 1024)
    assert device_imatrix(dev, O.Q4K, x4, np.tile(qw, 4), 1024) == want.tobytes() * 4
