"""Known answers for the oracle's weight quantizers BlockQ4K::from_float and
BlockQ6K::from_float (k_quants.rs:1470-1528, 2005-2075), the blocks and their
hand-derived bytes of tests/weight_kat.py.  Each case is checked byte for
byte; its construction is first checked to keep every final code clear of a
rounding boundary."""
import numpy as np
import pytest

import oracle as O
from weight_kat import CASES, code_margin


@pytest.mark.parametrize("name", sorted(CASES))
def test_weight_quantizer_known_answer(name):
    dt, case = CASES[name]
    x, want = case()
    assert code_margin(dt, x, want) < 0.3
    got = O.quantize(dt, x.reshape(1, 256))
    assert got.tobytes() == want.tobytes(), name


def test_known_answer_blocks_in_a_row():
    """The six blocks as consecutive superblocks of rows: from_float works per
    256 elements, so each keeps its bytes (Q6K's code buffer is reused across
    superblocks, k_quants.rs:2013-2017)."""
    for dt in (O.Q4K, O.Q6K):
        names = [n for n in sorted(CASES) if CASES[n][0] == dt]
        xs, ws = zip(*(CASES[n][1]() for n in names))
        x = np.concatenate(xs)[None]
        got = O.quantize(dt, np.concatenate([x, x[:, ::-1].copy()]))
        assert got[0].tobytes() == np.concatenate(ws).tobytes()


def test_q6k_search_window_improves_on_first_pass():
    """The codes make_qx_quants chooses on general data, observed directly.

    Group 0 is a grid group with step S (the block's largest scale); groups
    1..15 hold uniform data in (-S/4096, S/4096), so their scale bytes
    round(-128 s_g / S)
    are 0 and from_float keeps the search's own codes for them
    (k_quants.rs:2036-2040).  The refinement and the coordinate descent of
    utils.rs:62-226 only accept a change that raises
    (sum w x l)^2 / sum w l^2 with w = x^2, so the final codes score at least
    as high as the first pass l = round(-32 x / max) (max = the signed max |x|)
    does, evaluated here in float64; on this data the search does move codes in
    some groups; and the result is the descent's fixed point: for no element
    does the integer nearest its stationary code raise the score."""
    from blockref import q6k_fields
    from weight_kat import Q6K_S, round_half_away

    rng = np.random.default_rng(0)
    x = np.zeros(256, np.float32)
    q0 = rng.integers(-31, 32, 16)
    q0[4] = -32
    x[:16] = q0 * Q6K_S
    x[16:] = (rng.uniform(-1, 1, 240) * (Q6K_S / 4096)).astype(np.float32)
    b = O.quantize(O.Q6K, x.reshape(1, 256))
    _, sc, q = q6k_fields(b)
    sc, q = sc.reshape(16), q.reshape(256)
    assert sc[0] == -128 and np.all(sc[1:] == 0)
    moved = 0
    for g in range(1, 16):
        xg = x[16 * g:16 * g + 16].astype(np.float64)
        imax = int(np.argmax(np.abs(xg)))           # first index of the max |x|
        first = np.array([min(max(round_half_away(-32.0 * v / xg[imax]), -32), 31) for v in xg])
        final = q[16 * g:16 * g + 16]

        def score(l):
            w = xg * xg
            return (w * xg * l).sum() ** 2 / (w * l * l).sum()

        assert score(final) >= score(first) * (1 - 1e-6), g
        moved += int(np.any(final != first))
        # With the other codes fixed, the score as a function of code i,
        # (A + w_i x_i c)^2 / (B + w_i c^2) with A, B the other terms' sums,
        # has its stationary point at c* = x_i B / A (derivative zero).  The
        # descent stops when no element's nearest integer to c* (clamped to
        # [-32, 31]) raises the score: check that fixed point.
        w = xg * xg
        best = score(final)
        for i in range(16):
            A = (w * xg * final).sum() - w[i] * xg[i] * final[i]
            B = (w * final * final).sum() - w[i] * final[i] * final[i]
            if A <= 0:
                continue
            c = min(max(round_half_away(xg[i] * B / A), -32), 31)
            trial = final.copy()
            trial[i] = c
            assert score(trial) <= best * (1 + 1e-6), (g, i, c)
    assert moved >= 3
