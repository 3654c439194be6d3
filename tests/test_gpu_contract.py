"""Contract properties of the QMatMul seams on the GPU, through the C ABI.

* Bit stability: fuel declares the QMatMul path bit-identical on re-run on the
  same hardware (fuel-dispatch/src/fused.rs:1319-1330,
  bit_stable_on_same_hardware).  A call's kernels (frq_qmatmul_plan) and its
  output bits must therefore not depend on which calls ran before it in the
  process: the same calls in a fresh process, in this one after many others,
  and again after every other tile kernel has been planned and run, agree bit
  for bit.
* Thread safety: DynQuantizedStorage is Send + Sync
  (fuel-backend-contract/src/quantized.rs:29); two threads calling fwd on two
  storages of one device, with shapes that grow the device's workspace while
  the other thread's kernels may still use it, get the serial run's bits.
* The long-row K split of the wide Q4_K tiles (11008-column rows, 256-384
  activation rows, a ragged last row tile) against the oracle, f32 and f16.
"""
import ctypes as C
import json
import os
import subprocess
import sys
import threading

import numpy as np
import pytest

import fuel_amd as F
import oracle as O
from blockref import rel_err
from fuel_amd._native import check, lib

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TOL = 1e-3
TOL_F16 = TOL + 2.0 ** -11


def say(*a):
    print(*a, flush=True)


# (dtype, rows, n, k): Q4_K 4096x32000 at M = 32 (the 32-row wide tiles) and
# Q6_K 11008x4096 at M = 128 (plane kernel with a K split or wide tiles)
STABLE_CALLS = [(O.Q4K, 32, 32000, 4096), (O.Q6K, 128, 4096, 11008)]

# Computes the plan and the output digest of each call on a device; run as the
# first QMatMuls of a fresh process and inside the test process.  Inputs are
# generated on the device (Philox normals, device from_float), so both
# processes see the same bytes.
PROBE = r'''
import hashlib, json, sys
import numpy as np
import fuel_amd as F

def probe(dev, calls):
    out = []
    for dt, m, n, k in calls:
        x = F.fill_normal(dev, (m, k), seed=101, stream=m)
        wf = F.fill_normal(dev, (n, k), seed=102, stream=n, std=0.02)
        q = dev.qzeros(n * k, dt)
        q.quantize(wf)
        plan = F.qmatmul_plan(dev, dt, m, n, k, q.device_ptr())
        y, _ = q.fwd((n, k), x)
        digest = hashlib.sha256(y.numpy().tobytes()).hexdigest()
        out.append([list(plan), digest])
    return out

if __name__ == "__main__":
    dev = F.RocmDevice(0)
    print("RESULT " + json.dumps(probe(dev, json.loads(sys.argv[1]))), flush=True)
    dev.close()
'''


def _probe(dev, calls):
    ns = {}
    exec(compile(PROBE, "probe", "exec"), ns)
    return ns["probe"](dev, calls)


# every tile kernel kind and K split the plan can choose: Q4_K at 16-byte
# aligned and 4-byte aligned bases, Q6_K, 16..512 rows, short and long rows
OTHER_CALLS = [(dt, m, n, k) for dt in (O.Q4K, O.Q6K) for m in (16, 33, 64, 96, 128, 200, 384, 512)
               for n, k in ((4096, 4096), (11008, 4096), (4096, 11008), (1000, 2048))]


def test_plan_and_bits_do_not_depend_on_call_history(dev, tmp_path):
    calls = [list(c) for c in STABLE_CALLS]
    say("fresh process:", calls)
    env = dict(os.environ, PYTHONPATH=ROOT + os.pathsep + os.environ.get("PYTHONPATH", ""))
    script = tmp_path / "probe_plan.py"
    script.write_text(PROBE)
    r = subprocess.run([sys.executable, "-u", str(script), json.dumps(calls)], capture_output=True, text=True,
                       timeout=300, env=env, cwd=ROOT)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    fresh = json.loads([ln for ln in r.stdout.splitlines() if ln.startswith("RESULT ")][-1][7:])
    say("  fresh plans", [p for p, _ in fresh])
    here = _probe(dev, calls)
    say("  this process, after the earlier tests:", [p for p, _ in here])
    assert here == fresh
    # plan and run every other kind, on 16-byte aligned and 4-byte aligned Q4_K bases
    kinds = set()
    for dt, m, n, k in OTHER_CALLS:
        x = F.fill_normal(dev, (m, k), seed=7, stream=m)
        nb = n * (k // 256) * O.TYPE_SIZE[dt]
        buf = dev.alloc(((nb + 16) // 4,), np.uint32)
        for off in (0, 4) if dt == O.Q4K else (0,):
            kinds.add(F.qmatmul_plan(dev, dt, m, n, k, buf.ptr + off))
            out = dev.alloc((m, n), np.float32)
            check(lib().frq_memset(dev.handle, C.c_void_p(buf.ptr), 0, buf.nbytes))
            check(lib().frq_qmatmul(dev.handle, dt, 1, m, n, k, C.c_void_p(x.ptr), x.nbytes,
                                    C.c_void_p(buf.ptr + off), nb, C.c_void_p(out.ptr), out.nbytes))
    dev.synchronize()
    say("  planned and ran", len(kinds), "distinct (path, kind, ksplit):", sorted(kinds))
    assert len({kd for p, kd, _ in kinds if p == "tiled_mfma"}) >= 6
    again = _probe(dev, calls)
    assert again == fresh


def _threaded_storages(d, specs):
    out = []
    for dt, n, k in specs:
        wf = F.fill_normal(d, (n, k), seed=201, stream=n + k, std=0.02)
        q = d.qzeros(n * k, dt)
        q.quantize(wf)
        out.append(q)
    return out


# (dtype, n, k) per thread, and the row counts each thread cycles through: the
# tiled MFMA path grows the workspace (quantized rows + split-K partials) at
# 200 / 300 / 512 rows while the other thread's kernels are in flight
THREAD_SPECS = [(O.Q4K, 4096, 4096), (O.Q6K, 4096, 11008)]
THREAD_ROWS = [[1, 8, 64, 200, 512, 33, 2], [512, 2, 128, 48, 300, 1, 96]]


def test_two_threads_share_one_device(dev):
    rounds = 3
    # serial reference on the session device
    sq = _threaded_storages(dev, THREAD_SPECS)
    want = {}
    for t, (spec, rows) in enumerate(zip(THREAD_SPECS, THREAD_ROWS)):
        for m in rows:
            x = F.fill_normal(dev, (m, spec[2]), seed=300 + t, stream=m)
            y, _ = sq[t].fwd((spec[1], spec[2]), x)
            want[(t, m)] = y.numpy()
    # two threads on a fresh handle (an empty workspace that the calls grow)
    nd = F.RocmDevice(0)
    try:
        qs = _threaded_storages(nd, THREAD_SPECS)
        xs = {(t, m): F.fill_normal(nd, (m, THREAD_SPECS[t][2]), seed=300 + t, stream=m)
              for t in range(2) for m in THREAD_ROWS[t]}
        nd.synchronize()
        got = {}
        errors = []
        barrier = threading.Barrier(2)

        def work(t):
            try:
                n, k = THREAD_SPECS[t][1], THREAD_SPECS[t][2]
                barrier.wait()
                for r in range(rounds):
                    for m in THREAD_ROWS[t]:
                        y, _ = qs[t].fwd((n, k), xs[(t, m)])
                        got[(t, m, r)] = y.numpy()
            except Exception as e:  # reported by the main thread
                errors.append(repr(e))

        say("two threads on one device:", THREAD_SPECS, THREAD_ROWS, "x", rounds)
        th = [threading.Thread(target=work, args=(t,)) for t in range(2)]
        for t in th:
            t.start()
        for t in th:
            t.join(timeout=240)
        assert not any(t.is_alive() for t in th), "a thread did not finish"
        assert not errors, errors
        for (t, m, r), y in got.items():
            assert np.array_equal(y.view(np.uint32), want[(t, m)].view(np.uint32)), (t, m, r)
        assert len(got) == rounds * sum(len(r) for r in THREAD_ROWS)
    finally:
        nd.close()


@pytest.mark.parametrize("m", [256, 300, 384])
def test_wide_tiles_long_rows_k_split(dev, m):
    """Q4_K 11008x4096 at 256-384 rows: the wide-tile kernel with a K split
    (a ragged last 64-row tile at 300), f32 and f16 outputs, against the
    oracle."""
    k, n = 11008, 4096
    wq = O.quantize(O.Q4K, O.normal((n, k), seed=11, stream=2, std=0.02))
    x = O.normal((m, k), seed=12, stream=1)
    qs = dev.load_quantized(O.Q4K, wq.tobytes())
    path, kind, ks = F.qmatmul_plan(dev, O.Q4K, m, n, k, qs.device_ptr())
    say("wide long rows m", m, "plan", path, kind, ks)
    y, _ = qs.fwd((n, k), dev.from_numpy(x))
    err = rel_err(y.numpy(), O.matmul(O.Q4K, x, wq))
    say("  rel_err", err)
    assert err <= TOL
    x16 = O.f32_to_f16_bits(x)
    y16, _ = qs.fwd((n, k), dev.from_numpy(x16.view(np.float16)))
    err16 = rel_err(O.f16_bits_to_f32(y16.numpy().view(np.uint16)), O.f16_bits_to_f32(O.matmul_f16(O.Q4K, x16, wq)))
    say("  f16 rel_err", err16)
    assert err16 <= TOL_F16


@pytest.mark.parametrize("dt,m,k,n", [(O.Q4K, 3, 4096, 32000), (O.Q4K, 4, 4096, 16400), (O.Q4K, 8, 4096, 11008),
                                      (O.Q4K, 13, 4096, 11008), (O.Q4K, 16, 4096, 11008), (O.Q4K, 20, 4096, 11008),
                                      (O.Q4K, 28, 4096, 32000), (O.Q4K, 24, 11008, 4096), (O.Q4K, 29, 11008, 4096),
                                      (O.Q6K, 5, 4096, 32000), (O.Q6K, 16, 4096, 32000), (O.Q6K, 27, 2048, 25000),
                                      (O.Q6K, 26, 11008, 4096)])
def test_wide_tiles_3_to_32_rows(dev, dt, m, k, n):
    """Q4_K at 3-32 rows on the wide-tile kernel: 16 x 64 tiles with two
    wavefront groups (3-16 rows, ragged columns at 16400), 32 x 64 tiles with
    and without them (ragged rows), and rows of 11008 elements from 24 rows
    with a K split; Q6_K at 5-32 rows of >= 24576 columns on its wide-tile
    kernel in 16 x 64 and 32 x 64 tiles (ragged rows and columns), and rows of
    11008 elements from 24 rows on the 32-row plane tiles with a K split; f32
    and f16 outputs against the oracle."""
    wq = O.quantize(dt, O.normal((n, k), seed=13, stream=m, std=0.02))
    x = O.normal((m, k), seed=14, stream=m)
    qs = dev.load_quantized(dt, wq.tobytes())
    path, kind, ks = F.qmatmul_plan(dev, dt, m, n, k, qs.device_ptr())
    say("wide tiles dt", dt, "m", m, "k", k, "n", n, "plan", path, kind, ks)
    assert path == "tiled_mfma"
    y, _ = qs.fwd((n, k), dev.from_numpy(x))
    err = rel_err(y.numpy(), O.matmul(dt, x, wq))
    say("  rel_err", err)
    assert err <= TOL
    x16 = O.f32_to_f16_bits(x)
    y16, _ = qs.fwd((n, k), dev.from_numpy(x16.view(np.float16)))
    err16 = rel_err(O.f16_bits_to_f32(y16.numpy().view(np.uint16)), O.f16_bits_to_f32(O.matmul_f16(dt, x16, wq)))
    say("  f16 rel_err", err16)
    assert err16 <= TOL_F16
