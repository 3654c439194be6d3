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
