"""frq_qmatmul_noalloc: the QMatMul KernelRef entry point with its scratch in a
fixed per-GPU device array instead of an allocated workspace.  Through the C
ABI, against frq_qmatmul on the same inputs: bit-identical outputs (same
kernels, same plan) on two calls in a row, the second smaller than the first
(the array keeps the first call's contents), and a request beyond the array
refused with the workspace status, leaving the output untouched."""
import ctypes as C

import numpy as np
import pytest

import fuel_amd as F
import oracle as O
from fuel_amd._native import lib

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def run(dev, fn, dt, m, n, k, xd, wd, out):
    return fn(dev.handle, dt, 1, m, n, k, C.c_void_p(xd.ptr), xd.nbytes, C.c_void_p(wd.ptr), wd.nbytes,
              C.c_void_p(out.ptr), out.nbytes)


@pytest.fixture(scope="module")
def ndev():
    d = F.RocmDevice(0)
    yield d
    d.close()


# (dtype, m, n, k): the tiled MFMA path with its quantized rows, then a smaller
# skinny-path call, then a mat-vec row; Q8_0 through the skinny kernel
CALLS = [(O.Q4K, 512, 4096, 4096), (O.Q6K, 24, 1000, 4096), (O.Q4K, 1, 640, 2048), (O.Q8_0, 40, 512, 1024)]


def test_noalloc_matches_qmatmul_on_consecutive_calls(ndev):
    L = lib()
    for dt, m, n, k in CALLS:
        say("noalloc", dt, m, n, k)
        wq = O.quantize(dt, O.normal((n, k), seed=n + k, stream=3, std=0.02))
        x = O.normal((m, k), seed=m + k, stream=4)
        wd = ndev.from_numpy(np.frombuffer(wq.tobytes(), np.uint32))
        xd = ndev.from_numpy(x)
        want = ndev.alloc((m, n), np.float32)
        got = ndev.alloc((m, n), np.float32)
        F._native.check(run(ndev, L.frq_qmatmul, dt, m, n, k, xd, wd, want))
        F._native.check(run(ndev, L.frq_qmatmul_noalloc, dt, m, n, k, xd, wd, got))
        ndev.synchronize()
        assert np.array_equal(got.numpy().view(np.uint32), want.numpy().view(np.uint32))


def test_noalloc_refuses_beyond_its_scratch(ndev):
    L = lib()
    m, n, k = 4096, 64, 8192          # quantized rows ~38 MB > 32 MiB
    wd = ndev.alloc((n * (k // 256) * 144 // 4,), np.uint32)
    xd = ndev.alloc((m, k), np.float32)
    out = ndev.from_numpy(np.full((m, n), 7.0, np.float32))
    rc = run(ndev, L.frq_qmatmul_noalloc, O.Q4K, m, n, k, xd, wd, out)
    assert rc == 4, rc
    assert b"scratch" in L.frq_last_error()
    assert np.all(out.numpy() == 7.0)


# shapes whose split-K partials, in frq_qmatmul's plan, do not fit the fixed
# array beside the quantized rows: one row tile of very long rows (Q6_K at 128
# rows of K = 131072: 19 MB of quantized rows plus 8 splits of 2 MB partials;
# Q4_K wide tiles at 256 rows of K = 98304: 29 MB of rows plus 2-4 splits of
# 4 MB); the planner says which of them bind on this GPU
CAP_CANDIDATES = [(O.Q6K, 128, 4096, 131072), (O.Q4K, 256, 4096, 98304)]


def test_noalloc_lowered_split_within_tolerance(ndev):
    """When the plan's partials do not fit, frq_qmatmul_noalloc lowers the K
    split (frq_qmatmul_plan with noalloc = 1 shows it): the f32 sums are then
    added in another order, so the outputs agree with frq_qmatmul's within the
    path's tolerance (1e-3 of the output norm) rather than in bits."""
    L = lib()
    bound = 0
    for dt, m, n, k in CAP_CANDIDATES:
        wf = F.fill_normal(ndev, (n, k), seed=5, stream=n, std=0.02)
        q = ndev.qzeros(n * k, dt)
        q.quantize(wf)
        del wf
        reg = F.qmatmul_plan(ndev, dt, m, n, k, q.device_ptr())
        fixed = F.qmatmul_plan(ndev, dt, m, n, k, q.device_ptr(), noalloc=True)
        say("noalloc cap", dt, m, n, k, "plans", reg, fixed)
        if fixed == reg:
            continue
        assert fixed[0] == reg[0] == "tiled_mfma" and fixed[2] < reg[2]
        bound += 1
        xd = F.fill_normal(ndev, (m, k), seed=6, stream=m)
        nb = n * (k // 256) * O.TYPE_SIZE[dt]
        want = ndev.alloc((m, n), np.float32)
        got = ndev.alloc((m, n), np.float32)
        for fn, out in ((L.frq_qmatmul, want), (L.frq_qmatmul_noalloc, got)):
            F._native.check(fn(ndev.handle, dt, 1, m, n, k, C.c_void_p(xd.ptr), xd.nbytes, C.c_void_p(q.device_ptr()),
                               nb, C.c_void_p(out.ptr), out.nbytes))
        ndev.synchronize()
        a, b = got.numpy(), want.numpy()
        err = float(np.abs(a - b).max() / np.linalg.norm(b))
        say("  rel diff", err)
        assert np.all(np.isfinite(a)) and err <= 1e-3
    assert bound >= 1, "no candidate shape binds the fixed scratch"
