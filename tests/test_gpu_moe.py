"""GPU parity of the MoE mul_mat_id path against the CPU oracle, through the C ABI.

Bit-exact: routing ids (descending logit, ties to the lower expert id,
lazy_nn/moe.rs:90-127 with byte_kernels.rs:8246-8261), expert_offsets,
sorted_token_ids and the (token, slot) entry of each sorted position
(moe_routing.rs:334-360).  f32: routing weights within a few ulp (device
expf), expert outputs max |y_gpu - y_cpu| <= 1e-3 * ||y_cpu||_2 against the
oracle's expert FFN (lazy_nn/moe.rs:204-235, 296-348) on the same blocks.
"""
import functools

import numpy as np
import pytest

import fuel_amd as F
import oracle as O
from blockref import rel_err

pytestmark = pytest.mark.gpu

TOL = 1e-3


def say(*a):
    print(*a, flush=True)


def route_both(dev, logits, k):
    want = O.moe_route(logits, k)
    got = F.moe_route(dev, dev.from_numpy(logits), k)
    return want, got


def assert_route_equal(want, got, exact_w=False):
    ids, w, off, sid, slot = want
    gids, gw, goff, gsid, gslot = got
    np.testing.assert_array_equal(gids, ids)
    np.testing.assert_array_equal(goff, off)
    np.testing.assert_array_equal(gsid, sid)
    np.testing.assert_array_equal(gslot, slot)
    if exact_w:
        np.testing.assert_array_equal(gw, w)
    else:
        np.testing.assert_allclose(gw, w, rtol=2e-6, atol=1e-7, equal_nan=True)


def test_moe_route_known_answer(dev):
    """moe_routing.rs:372-392: [[3,1,0,0],[0,0,2,4]] top-2 -> {0,1}, {3,2}."""
    say("moe_route known answer")
    logits = np.array([[3, 1, 0, 0], [0, 0, 2, 4]], np.float32)
    want, got = route_both(dev, logits, 2)
    assert got[0].tolist() == [[0, 1], [3, 2]]
    assert_route_equal(want, got)


@pytest.mark.parametrize("t,e,k", [(1, 128, 8), (16, 128, 8), (512, 128, 8), (37, 64, 1), (9, 300, 20),
                                   (3, 1000, 64), (2000, 128, 8)])
def test_moe_route_bit_exact(dev, t, e, k):
    say("moe_route", t, e, k)
    logits = O.normal((t, e), seed=t * 1000 + e, stream=7)
    want, got = route_both(dev, logits, k)
    assert_route_equal(want, got)


def test_moe_route_ties_and_specials(dev):
    """Equal logits go to the lower expert id; -inf, NaN and masked picks
    follow the sequential first-max scan."""
    say("moe_route ties")
    e = 70
    rows = [np.zeros(e), np.full(e, 2.5), np.arange(e) % 4, -np.arange(e) % 3]
    r = O.normal((1, e), seed=5, stream=1)[0].astype(np.float64)
    r[[5, 9, 66]] = r.max() + 1.0                   # a three-way tie at the top
    rows.append(r)
    r = np.full(e, -np.inf)
    r[[3, 40]] = [1.0, -2.0]                        # fewer finite values than k
    rows.append(r)
    r = O.normal((1, e), seed=6, stream=1)[0].astype(np.float64)
    r[[2, 30]] = np.nan                             # NaN off the first slot: never picked
    rows.append(r)
    logits = np.stack(rows).astype(np.float32)
    want, got = route_both(dev, logits, 6)
    assert_route_equal(want, got)
    assert got[0][0].tolist() == [0, 1, 2, 3, 4, 5]


def test_moe_route_nan_first_slot(dev):
    """A NaN logit in slot 0 is never displaced by the scan: every pick is
    expert 0 (duplicate entries keep slot order in the batches)."""
    say("moe_route nan first")
    logits = O.normal((3, 16), seed=8, stream=1)
    logits[1, 0] = np.nan
    want, got = route_both(dev, logits, 4)
    assert got[0][1].tolist() == [0, 0, 0, 0]
    assert_route_equal(want, got)


# ---- indexed mat-vec (DynQuantizedStorage::indexed_moe_forward) ----

@functools.lru_cache(maxsize=None)
def experts(dt, e, n, k, seed=21):
    return O.quantize(dt, O.normal((e, n, k), seed=seed, stream=3, std=0.02))


@pytest.mark.parametrize("dt,e,n,k", [(O.Q4K, 8, 512, 2048), (O.Q6K, 5, 256, 768), (O.Q8_0, 6, 384, 1024)])
@pytest.mark.parametrize("per_slot", [False, True])
def test_indexed_moe_forward(dev, dt, e, n, k, per_slot):
    say("indexed_moe_forward", dt, e, n, k, per_slot)
    t, topk = 7, 3
    w = experts(dt, e, n, k)
    rng = np.random.default_rng(dt * 100 + e)
    ids = rng.integers(0, e, size=(t, topk)).astype(np.int32)
    x = O.normal((t, topk, k) if per_slot else (t, k), seed=31, stream=e)
    q = dev.load_quantized(dt, w.tobytes())
    y, shape = q.indexed_moe_forward((e, n, k), dev.from_numpy(x), dev.from_numpy(ids))
    assert shape == (t, topk, n)
    got = y.numpy()
    for r in range(t):
        for s in range(topk):
            xr = x[r, s] if per_slot else x[r]
            want = O.matmul(dt, xr[None], w[ids[r, s]])[0]
            assert rel_err(got[r, s], want) < TOL, (r, s)


def test_indexed_moe_forward_bad_id_gives_nan_row(dev):
    say("indexed_moe_forward bad id")
    e, n, k = 4, 256, 512
    w = experts(O.Q4K, e, n, k)
    q = dev.load_quantized(O.Q4K, w.tobytes())
    ids = np.array([[1, 4], [-1, 2]], np.int32)
    x = O.normal((2, k), seed=3, stream=3)
    got = q.indexed_moe_forward((e, n, k), dev.from_numpy(x), dev.from_numpy(ids))[0].numpy()
    assert np.isnan(got[0, 1]).all() and np.isnan(got[1, 0]).all()
    assert rel_err(got[0, 0], O.matmul(O.Q4K, x[:1], w[1])[0]) < TOL
    assert rel_err(got[1, 1], O.matmul(O.Q4K, x[1:], w[2])[0]) < TOL
    with pytest.raises(F.FuelRocmError):
        q.indexed_moe_forward((e + 1, n, k), dev.from_numpy(x), dev.from_numpy(ids))


# ---- the expert layer ----

def device_experts(dev, dt, e, rows, cols, seed, stream):
    """Expert weights N(0, 0.02) generated and quantized on the device; the
    oracle is handed the same block bytes."""
    w32 = F.fill_normal(dev, (e, rows, cols), seed, stream, 0.0, 0.02)
    q = dev.qzeros(e * rows * cols, dt)
    q.quantize(w32)
    w32.free()
    blocks = np.frombuffer(q.data(), dtype=O.BLOCK_DTYPE[dt]).reshape(e, rows, cols // O.BLOCK_SIZE[dt])
    return q, blocks


@pytest.mark.parametrize("t,d,ffn,e,k,dt", [
    (1, 2048, 768, 128, 8, O.Q4K),        # Qwen3-MoE-style expert layer, decode
    (16, 2048, 768, 128, 8, O.Q4K),       # one routed entry per expert: the indexed mat-vec
    (17, 2048, 768, 128, 8, O.Q4K),       # just above it: the grouped int8-MFMA tiles
    (3, 256, 512, 6, 2, O.Q4K),           # entries == experts on a small layer
    (512, 2048, 768, 128, 8, O.Q4K),
    (5, 256, 512, 6, 2, O.Q4K),
    (9, 512, 256, 10, 3, O.Q6K),
    (11, 256, 512, 7, 2, O.Q8_0),
    (2, 256, 8192, 4, 2, O.Q4K),          # an entry's blocks past 32 lanes: indexed down + combine kernel
    (1, 512, 256, 300, 16, O.Q4K),        # 16 entries: four passes of the fused down + combine
])
def test_moe_ffn(dev, t, d, ffn, e, k, dt):
    say("moe_ffn", t, d, ffn, e, k, dt)
    seed = 500 + t
    wg, bg = device_experts(dev, dt, e, ffn, d, seed, 3)
    wu, bu = device_experts(dev, dt, e, ffn, d, seed, 4)
    wd, bd = device_experts(dev, dt, e, d, ffn, seed, 5)
    x = O.normal((t, d), seed=seed, stream=1)
    logits = O.normal((t, e), seed=seed, stream=2)
    ids, w, *_ = O.moe_route(logits, k)
    want = O.moe_ffn(dt, x, ids, w, bg, bu, bd)
    got = F.moe_ffn(dev, dt, dev.from_numpy(x), dev.from_numpy(logits), wg, wu, wd, ffn, k).numpy()
    err = rel_err(got, want)
    say("  rel_err", err)
    assert err < TOL


def test_moe_ffn_errors(dev):
    x = dev.alloc((2, 256), np.float32)
    logits = dev.alloc((2, 4), np.float32)
    for bad in [dict(k=5), dict(k=0)]:
        with pytest.raises(F.FuelRocmError):
            F.moe_ffn(dev, O.Q4K, x, logits, 0, 0, 0, 256, bad["k"])
    with pytest.raises(F.FuelRocmError):  # ffn not a multiple of the block
        F.moe_ffn(dev, O.Q4K, x, logits, 0, 0, 0, 100, 2)
