"""Pins of the oracle's MoE routing and expert FFN (CPU only).

Routing follows LazyMoeRouter::route (fuel-core/src/lazy_nn/moe.rs:90-127):
k rounds of argmax (first index on ties, byte_kernels.rs:8246-8261) and a
softmax over the picked logits; batches follow build_expert_batches
(fuel-inference/src/moe_routing.rs:334-360).  Known answer:
moe_routing.rs:372-392; invariants: lazy_nn/moe.rs:423-470 (k distinct ids,
weights sum to 1); brute-force sort on small T x E.
"""
import numpy as np

import oracle as O
from blockref import rel_err


def test_route_known_answer_top2():
    ids, w, off, sorted_ids, slot = O.moe_route(np.array([[3, 1, 0, 0], [0, 0, 2, 4]], np.float32), 2)
    assert ids.tolist() == [[0, 1], [3, 2]]
    assert np.allclose(w.sum(1), 1.0, atol=1e-6)
    assert off.tolist() == [0, 1, 2, 3, 4]
    assert sorted_ids.tolist() == [0, 0, 1, 1]
    assert slot.tolist() == [0, 1, 3, 2]


def test_route_tie_goes_to_lower_expert():
    ids, *_ = O.moe_route(np.array([[1, 5, 5, 2, 5]], np.float32), 3)
    assert ids.tolist() == [[1, 2, 4]]


def test_route_brute_force():
    t, e, k = 40, 16, 4
    logits = O.normal((t, e), seed=1, stream=3)
    ids, w, off, sorted_ids, slot = O.moe_route(logits, k)
    want = np.argsort(-logits, axis=1, kind="stable")[:, :k]
    assert np.array_equal(ids, want)
    assert all(len(set(r)) == k for r in ids.tolist())
    picked = np.take_along_axis(logits, ids, 1).astype(np.float64)
    sm = np.exp(picked - picked.max(1, keepdims=True))
    assert np.allclose(w, sm / sm.sum(1, keepdims=True), rtol=1e-6, atol=1e-7)
    # expert-major, token-ascending batches
    for ex in range(e):
        toks = sorted_ids[off[ex]:off[ex + 1]]
        assert toks.tolist() == [r for r in range(t) if ex in ids[r]]
        assert np.all(ids.reshape(-1)[slot[off[ex]:off[ex + 1]]] == ex)
    assert off[-1] == t * k


def test_moe_ffn_matches_dense_float_reference():
    t, d, ffn, e, k = 5, 256, 512, 6, 2
    x = O.normal((t, d), seed=2, stream=1)
    logits = O.normal((t, e), seed=2, stream=2)
    ids, w, *_ = O.moe_route(logits, k)
    wg = O.quantize(O.Q4K, O.normal((e, ffn, d), seed=2, stream=3, std=0.02))
    wu = O.quantize(O.Q4K, O.normal((e, ffn, d), seed=2, stream=4, std=0.02))
    wd = O.quantize(O.Q4K, O.normal((e, d, ffn), seed=2, stream=5, std=0.02))
    got = O.moe_ffn(O.Q4K, x, ids, w, wg, wu, wd)
    ref = np.zeros((t, d))
    G, U, D = (O.dequantize(O.Q4K, a).astype(np.float64) for a in (wg, wu, wd))
    for r in range(t):
        for s in range(k):
            ex = ids[r, s]
            g = G[ex] @ x[r]
            u = U[ex] @ x[r]
            h = g / (1 + np.exp(-g)) * u
            ref[r] += w[r, s] * (D[ex] @ h)
    assert rel_err(got, ref) < 2e-2
