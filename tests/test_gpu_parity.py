"""GPU parity of the HIP path against the CPU oracle, through the C ABI.

Bit-exact: activation int8 quants (Q8K / Q8_0 blocks), per-block integer dot
sums, dequantized values.  f32 outputs: max |y_gpu - y_cpu| <= 1e-3 * ||y_cpu||_2
against the oracle's restatement of fuel's CPU
matmul<T> (AVX2 vec_dot, k_quants.rs:2284-2331) on the same seeded inputs.
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


@functools.lru_cache(maxsize=None)
def weights(dt, n, k, seed=11):
    w = O.normal((n, k), seed=seed, stream=2, std=0.02)
    return O.quantize(dt, w)


@functools.lru_cache(maxsize=None)
def acts(m, k, seed=11):
    return O.normal((m, k), seed=seed, stream=1)


def as_u32(blocks: np.ndarray) -> np.ndarray:
    raw = np.frombuffer(blocks.tobytes(), np.uint8)
    assert raw.size % 4 == 0
    return raw.view(np.uint32)


# ---- activation quantizers (bit-exact) ----

def special_rows(k):
    rows = [np.arange(k, dtype=np.float32) % 256 - 128,            # integer closed form
            np.zeros(k, np.float32)]                                # zero blocks
    t = np.zeros(k, np.float32)
    t[3::256], t[10::256] = -5.0, 5.0                               # first-index ties
    rows.append(t)
    return np.stack(rows)


@pytest.mark.parametrize("m,k", [(1, 4096), (3, 11008), (5, 256)])
def test_quantize_q8k_bit_exact(dev, m, k):
    say("quantize_q8k", m, k)
    x = np.concatenate([acts(m, k), special_rows(k)])
    want = O.quantize(O.Q8K, x)
    xd = dev.from_numpy(x)
    got = F.quantize_q8k(dev, xd, x.shape[0], k)
    assert got.tobytes() == want.tobytes()


@pytest.mark.parametrize("m,k", [(1, 4096), (3, 11008), (2, 96)])
def test_quantize_q8_0_bit_exact(dev, m, k):
    say("quantize_q8_0", m, k)
    x = np.concatenate([acts(m, k), special_rows(k)])
    want = O.quantize(O.Q8_0, x)
    got = F.quantize_q8_0(dev, dev.from_numpy(x), x.shape[0], k)
    assert got.tobytes() == want.tobytes()


# ---- integer dot sums (bit-exact) ----

@pytest.mark.parametrize("dt", [O.Q4K, O.Q6K, O.Q8_0])
@pytest.mark.parametrize("m,n,k", [(2, 37, 1024), (1, 8, 11008)])
def test_block_isums_bit_exact(dev, dt, m, n, k):
    say("block_isums", dt, m, n, k)
    wq = weights(dt, n, k)
    x = acts(m, k)
    aq = O.quantize(O.VEC_DOT_TYPE[dt], x)
    want_i, want_m = O.block_isums(dt, wq, aq)
    wd = dev.load_quantized(dt, wq.tobytes())
    xd = dev.from_numpy(x)
    isum = dev.alloc((m, n, wq.shape[1]), np.int32)
    msum = dev.alloc((m, n, wq.shape[1]), np.int32)
    import ctypes as C
    from fuel_amd._native import check, lib
    check(lib().frq_block_isums(dev.handle, dt, m, n, k, C.c_void_p(wd.device_ptr()), C.c_void_p(xd.ptr),
                                C.c_void_p(isum.ptr), C.c_void_p(msum.ptr)))
    assert np.array_equal(isum.numpy(), want_i)
    assert np.array_equal(msum.numpy(), want_m)


# ---- f32 outputs through the KernelRef seam ----

SHAPES_7B = [(4096, 4096), (4096, 11008), (11008, 4096), (4096, 32000)]


@pytest.mark.parametrize("dt", [O.Q4K, O.Q6K])
@pytest.mark.parametrize("k,n", SHAPES_7B)
def test_qmatmul_m1_7b_shapes(dev, dt, k, n):
    say("qmatmul m=1", dt, k, n)
    wq = weights(dt, n, k)
    x = acts(1, k)
    want = O.matmul(dt, x, wq)
    act = dev.from_numpy(x)
    w = dev.from_numpy(as_u32(wq))
    out = dev.alloc((1, n), np.float32)
    F.qmatmul_f32_rocm_wrapper([act, w], [out], F.QMatMulParams(dt, 1, 1, n, k))
    got = out.numpy()
    err = rel_err(got, want)
    say("  rel_err", err)
    assert err <= TOL


@pytest.mark.parametrize("dt", [O.Q4K, O.Q6K, O.Q8_0])
@pytest.mark.parametrize("m,k,n", [(2, 4096, 4096), (3, 4096, 1000), (8, 4096, 4096), (15, 11008, 4096),
                                   (5, 11008, 776), (9, 2048, 300), (16, 256, 40), (24, 4096, 1000),
                                   (32, 11008, 4096), (2, 1024, 333), (3, 4096, 8200), (4, 2048, 9001),
                                   (2, 4096, 32000), (6, 4096, 8200), (4, 4096, 1000)])
def test_qmatmul_small_batch(dev, dt, m, k, n):
    """2 <= M <= 32 rows: the skinny int8-MFMA kernel (rows quantized once,
    each weight block read once per 32-row group, K split over the
    workgroup's wavefronts) or the mat-vec with several rows per workgroup —
    2 rows of the k-quants with K <= 4096 and 3-4 rows of wide ones (the
    8200- and 9001-column cases); Q8_0 at K = 4096 with 2-4 rows, and 5-8 rows
    of wide matrices in two row groups; Q4_K (16-byte aligned) on the wide-tile
    int8-MFMA kernel for 5+ rows of >= 8192 columns and 24+ rows of 11008
    elements: within the tolerance of the oracle,
    and independent of the other rows of the batch: the same rows in another
    order give every row the same bits."""
    say("small batch", dt, m, k, n)
    wq = weights(dt, n, k)
    x = acts(m, k, seed=m)
    want = O.matmul(dt, x, wq)
    w = dev.from_numpy(as_u32(wq))
    xd = dev.from_numpy(x)
    out = dev.alloc((m, n), np.float32)
    F.qmatmul_f32_rocm_wrapper([xd, w], [out], F.QMatMulParams(dt, 1, m, n, k))
    got = out.numpy()
    err = rel_err(got, want)
    say("  rel_err", err)
    assert err <= TOL
    rolled = np.ascontiguousarray(np.roll(x, 1, axis=0))
    out2 = dev.alloc((m, n), np.float32)
    F.qmatmul_f32_rocm_wrapper([dev.from_numpy(rolled), w], [out2], F.QMatMulParams(dt, 1, m, n, k))
    np.testing.assert_array_equal(np.roll(out2.numpy(), -1, axis=0).view(np.uint32), got.view(np.uint32))
    if m == 2 and k <= 4096 and (dt != O.Q8_0 or k == 4096):
        # (two rows of the mat-vec: each row is the one-row call's, bit for bit)
        one = dev.alloc((1, n), np.float32)
        for r in range(2):
            F.qmatmul_f32_rocm_wrapper([dev.from_numpy(np.ascontiguousarray(x[r:r + 1])), w], [one],
                                       F.QMatMulParams(dt, 1, 1, n, k))
            np.testing.assert_array_equal(one.numpy()[0].view(np.uint32), got[r].view(np.uint32))


@pytest.mark.parametrize("m", [16, 32, 100])
def test_qmatmul_q8_0_batched(dev, m):
    """Q8_0 (no tiled MFMA kernel) at 16 or more rows: the skinny int8-MFMA
    kernel, one weight pass per 32-row group, against the oracle at
    4096 x 4096."""
    say("q8_0 batched", m)
    k = n = 4096
    wq = weights(O.Q8_0, n, k)
    x = acts(m, k)
    want = O.matmul(O.Q8_0, x, wq)
    out = dev.alloc((m, n), np.float32)
    F.qmatmul_f32_rocm_wrapper([dev.from_numpy(x), dev.from_numpy(as_u32(wq))], [out],
                               F.QMatMulParams(O.Q8_0, 1, m, n, k))
    err = rel_err(out.numpy(), want)
    say("  rel_err", err)
    assert err <= TOL


def test_qmatmul_q8_0_config1(dev):
    # Q8_0 QMatMul, x [1,4096] ~ N(0,1), W [4096,4096] ~ N(0,0.02)
    k = n = 4096
    wq = weights(O.Q8_0, n, k)
    x = acts(1, k)
    want = O.matmul(O.Q8_0, x, wq)
    out = dev.alloc((1, n), np.float32)
    F.qmatmul_f32_rocm_wrapper([dev.from_numpy(x), dev.from_numpy(as_u32(wq))], [out],
                               F.QMatMulParams(O.Q8_0, 1, 1, n, k))
    assert rel_err(out.numpy(), want) <= TOL


@pytest.mark.parametrize("dt", [O.Q4K, O.Q6K])
@pytest.mark.parametrize("m,n,k", [(1, 1, 512), (1, 2, 256), (1, 6, 768), (2, 5, 1024), (1, 7, 1536), (3, 6, 1792),
                                   (1, 9, 2048), (4, 2049, 512)])
def test_qmatmul_short_rows(dev, dt, m, n, k):
    # rows of at most 8 superblocks go two or four to a wavefront step: row
    # counts that leave a group part-filled, groups past the last row; the
    # output starts as NaN so an unwritten row fails (n * k/256 even: the
    # weights go in as u32 words, and a Q6_K block is 210 bytes)
    say("qmatmul short rows", dt, m, n, k)
    wq = weights(dt, n, k)
    x = acts(m, k)
    want = O.matmul(dt, x, wq)
    out = dev.from_numpy(np.full((m, n), np.nan, np.float32))
    F.qmatmul_f32_rocm_wrapper([dev.from_numpy(x), dev.from_numpy(as_u32(wq))], [out],
                               F.QMatMulParams(dt, 1, m, n, k))
    got = out.numpy()
    assert np.isfinite(got).all()
    for r in range(m):
        assert rel_err(got[r], want[r]) <= TOL, r


@pytest.mark.parametrize("dt", [O.Q4K, O.Q6K, O.Q8_0])
def test_qmatmul_batched_small(dev, dt):
    batch, m, n, k = 2, 3, 40, 512
    wq = weights(dt, n, k)
    x = acts(batch * m, k)
    want = O.matmul(dt, x, wq)
    out = dev.alloc((batch, m, n), np.float32)
    F.qmatmul_f32_rocm_wrapper([dev.from_numpy(x.reshape(batch, m, k)), dev.from_numpy(as_u32(wq))], [out],
                               F.QMatMulParams(dt, batch, m, n, k))
    assert rel_err(out.numpy().reshape(batch * m, n), want) <= TOL


def test_q6k_all_ones_against_cpu_path(dev):
    # fuel-dispatch/src/pipelined.rs:10073-10139: n=2, k=256, all-ones W, act = i/100
    n, k = 2, 256
    wq = O.quantize(O.Q6K, np.ones((n, k), np.float32))
    x = (np.arange(1, k + 1, dtype=np.float32) / 100.0).reshape(1, k)
    want = O.matmul(O.Q6K, x, wq)
    out = dev.alloc((1, n), np.float32)
    F.qmatmul_f32_rocm_wrapper([dev.from_numpy(x), dev.from_numpy(as_u32(wq))], [out],
                               F.QMatMulParams(O.Q6K, 1, 1, n, k))
    assert rel_err(out.numpy(), want) <= 1e-6


# ---- DynQuantizedStorage seam ----

@pytest.mark.parametrize("dt", [O.Q4K, O.Q6K, O.Q8_0])
def test_qstorage_fwd_dequantize_data(dev, dt):
    n, k = 33, 768
    wq = weights(dt, n, k)
    qs = dev.load_quantized(dt, wq.tobytes())
    assert qs.dtype() == dt and qs.block_size() == O.BLOCK_SIZE[dt]
    assert qs.storage_size_in_bytes() == wq.nbytes
    assert qs.data() == wq.tobytes()
    x = acts(4, k).reshape(2, 2, k)
    y, shape = qs.fwd((n, k), dev.from_numpy(x))
    assert shape == (2, 2, n)
    assert rel_err(y.numpy().reshape(4, n), O.matmul(dt, x.reshape(4, k), wq)) <= TOL
    deq = qs.dequantize(n * k).numpy()
    assert np.array_equal(deq.view(np.uint32), O.dequantize(dt, wq).reshape(-1).view(np.uint32))
    deq16 = qs.dequantize_f16(n * k).numpy()
    assert np.array_equal(deq16, O.dequantize(dt, wq).reshape(-1).astype(np.float16).view(np.uint16))


# f16 output rounding adds at most half an f16 ulp (2^-11 relative) per element
TOL_F16 = TOL + 2.0 ** -11


@pytest.mark.parametrize("dt", [O.Q4K, O.Q6K, O.Q8_0])
@pytest.mark.parametrize("m,n,k", [(1, 300, 4096), (3, 64, 1024), (32, 1024, 4096), (512, 256, 2048),
                                   (16, 8200, 1024)])
def test_qstorage_fwd_f16(dev, dt, m, n, k):
    """matmul_f16 through fwd: f16 rows in, f16 rows out.  Against the oracle's
    matmul_f16 within the f32 tolerance plus the output rounding, and bit-exact
    against the device's own f32 path on the widened rows rounded by the
    oracle's f16::from_f32 (same kernels, same sums: only the I/O differs)."""
    say("fwd f16", dt, m, n, k)
    wq = weights(dt, n, k)
    qs = dev.load_quantized(dt, wq.tobytes())
    x16 = O.f32_to_f16_bits(acts(m, k))
    x32 = O.f16_bits_to_f32(x16)
    y16, shape = qs.fwd((n, k), dev.from_numpy(x16.view(np.float16)))
    assert shape == (m, n) and y16.dtype == np.float16
    got = y16.numpy().view(np.uint16)
    want = O.matmul_f16(dt, x16, wq)
    err = rel_err(O.f16_bits_to_f32(got), O.f16_bits_to_f32(want))
    say("  rel_err", err)
    assert err <= TOL_F16
    y32, _ = qs.fwd((n, k), dev.from_numpy(x32))
    assert np.array_equal(got, O.f32_to_f16_bits(y32.numpy()))


def test_qzeros_and_errors(dev):
    z = dev.qzeros(512, O.Q4K)
    assert z.data() == bytes(2 * 144)
    with pytest.raises(F.FuelRocmError) as e:
        dev.qzeros(100, O.Q4K)
    assert e.value.status == 2
    with pytest.raises(F.FuelRocmError) as e:
        dev.load_quantized(O.Q6K, bytes(211))
    assert e.value.status == 2
    with pytest.raises(F.FuelRocmError) as e:
        dev.load_quantized(2, bytes(18))      # Q4_0: not this backend's format
    assert e.value.status == 3
    qs = dev.load_quantized(O.Q4K, weights(O.Q4K, 4, 512).tobytes())
    with pytest.raises(F.FuelRocmError):
        qs.fwd((4, 512), dev.from_numpy(np.zeros((1, 256), np.float32)))   # k mismatch


def test_kernelref_validation(dev):
    wq = weights(O.Q4K, 4, 512)
    w = dev.from_numpy(as_u32(wq))
    act = dev.from_numpy(np.zeros((1, 512), np.float32))
    out = dev.alloc((1, 4), np.float32)
    bad = [F.QMatMulParams(O.Q4K, 1, 1, 4, 500),     # k not a block multiple
           F.QMatMulParams(O.Q4K, 1, 1, 5, 512),     # weight bytes mismatch
           F.QMatMulParams(O.Q4K, 2, 1, 4, 512)]     # activation bytes mismatch
    for p in bad:
        with pytest.raises(F.FuelRocmError) as e:
            F.qmatmul_f32_rocm_wrapper([act, w], [out], p)
        assert e.value.status == 2
    # zero m is a no-op that leaves the output untouched
    sentinel = np.full((1, 4), 7.0, np.float32)
    out.copy_from(sentinel)
    empty = dev.alloc((1,), np.float32)
    import ctypes as C
    from fuel_amd._native import lib
    assert lib().frq_qmatmul(dev.handle, O.Q4K, 1, 0, 4, 512, C.c_void_p(empty.ptr), 0, C.c_void_p(w.ptr),
                             w.nbytes, C.c_void_p(empty.ptr), 0) == 0
    assert np.array_equal(out.numpy(), sentinel)


# ---- device from_float (DynQuantizedStorage::quantize) and synthetic inputs ----

def weight_rows(k):
    rows = [np.zeros(k, np.float32), np.ones(k, np.float32), np.full(k, -0.75, np.float32),
            (np.arange(k, dtype=np.float32) % 97 - 48) / 64]
    spiky = np.zeros(k, np.float32)
    spiky[::37] = 3.0
    spiky[5::41] = -7.0
    rows.append(spiky)
    return np.stack(rows)


@pytest.mark.parametrize("dt", [O.Q4K, O.Q6K, O.Q8_0])
def test_device_quantize_bit_exact(dev, dt):
    say("device from_float", dt)
    k = 2048
    w = np.concatenate([O.normal((64, k), seed=21, stream=5, std=0.02), weight_rows(k),
                        O.normal((3, k), seed=22, stream=6, std=3.0)])
    want = O.quantize(dt, w)
    q = dev.qzeros(w.size, dt)
    q.quantize(dev.from_numpy(w))
    got = np.frombuffer(q.data(), O.BLOCK_DTYPE[dt]).reshape(want.shape)
    bad = np.nonzero(got.view(np.uint8).reshape(got.size, -1) != want.view(np.uint8).reshape(want.size, -1))
    assert got.tobytes() == want.tobytes(), f"first differing blocks {np.unique(bad[0])[:8]}"


def test_device_quantize_known_answers(dev):
    """The hand-derived known-answer blocks of weight_kat.py (grid-exact
    sub-blocks, clamps, ties, saturation, zero blocks) through the device
    from_float, byte for byte against the hand results."""
    from weight_kat import CASES

    for dt in (O.Q4K, O.Q6K):
        names = [n for n in sorted(CASES) if CASES[n][0] == dt]
        say("device from_float known answers", names)
        xs, ws = zip(*(CASES[n][1]() for n in names))
        x = np.concatenate(xs)[None]
        q = dev.qzeros(x.size, dt)
        q.quantize(dev.from_numpy(x))
        assert q.data() == np.concatenate(ws).tobytes()


def test_random_bits_bit_exact(dev):
    seed, base, stream = 0xDEADBEEF12345678, 3, 9
    got = F.fill_random_bits(dev, 1001, 7, seed, base, stream).numpy()
    assert np.array_equal(got, O.random_bits(1001, 7, seed, base, stream))


def test_normal_matches_host_generator(dev):
    got = F.fill_normal(dev, (3, 1000), 5, 2, 0.0, 0.02).numpy()
    want = O.normal((3, 1000), seed=5, stream=2, std=0.02)
    ulp = np.spacing(np.abs(want).astype(np.float32))
    assert np.all(np.abs(got - want) <= ulp)


# ---- batched / prefill: int8 MFMA path (M >= 16) ----

@pytest.mark.parametrize("dt", [O.Q4K, O.Q6K])
@pytest.mark.parametrize("m", [16, 32, 128, 512])
def test_qmatmul_mfma_rows(dev, dt, m):
    say("mfma dt", dt, "m", m)
    k, n = 4096, 4096
    wq = weights(dt, n, k)
    x = acts(m, k)
    want = O.matmul(dt, x, wq)
    out = dev.alloc((m, n), np.float32)
    F.qmatmul_f32_rocm_wrapper([dev.from_numpy(x), dev.from_numpy(as_u32(wq))], [out],
                               F.QMatMulParams(dt, 1, m, n, k))
    err = rel_err(out.numpy(), want)
    say("  rel_err", err)
    assert err <= TOL


@pytest.mark.parametrize("dt", [O.Q4K, O.Q6K])
@pytest.mark.parametrize("k,n", SHAPES_7B)
@pytest.mark.parametrize("m", [16, 24, 32, 48, 96, 128, 160, 200, 512])
def test_qmatmul_mfma_7b_shapes(dev, dt, k, n, m):
    """M = 32 / 128 / 512 rows at the four 7B shapes (the
    43-superblock rows of K = 11008, split K, the LDS-DMA staging), 16 / 24
    rows (the tiled kernel's partly empty 32-row tiles for the wide matrices,
    the skinny kernel at N = 4096), and 48 / 96 / 160 / 200 rows: Q4_K's 32 x
    64 and 64 x 128 wide tiles with and without a K split in memory, with one
    or two wavefront groups splitting K inside the workgroup (4096x4096 at 48
    and 128 rows, 512 rows of 4096x4096 and 11008x4096; ragged row tiles, a
    4096x11008 grid just past one workgroup per CU at 160 rows), Q6_K's
    partly empty 128-row plane tiles at 96 rows and its wide tiles at 48 rows
    of 4096x32000, against the oracle."""
    say("mfma", dt, "m", m, k, n)
    wq = weights(dt, n, k)
    x = acts(m, k)
    want = O.matmul(dt, x, wq)
    out = dev.alloc((m, n), np.float32)
    F.qmatmul_f32_rocm_wrapper([dev.from_numpy(x), dev.from_numpy(as_u32(wq))], [out],
                               F.QMatMulParams(dt, 1, m, n, k))
    err = rel_err(out.numpy(), want)
    say("  rel_err", err)
    assert err <= TOL


@pytest.mark.parametrize("dt", [O.Q4K, O.Q6K])
@pytest.mark.parametrize("m,n,k", [(130, 8200, 256), (200, 4100, 512), (333, 3000, 768), (129, 9000, 1280)])
def test_qmatmul_wide_tiles(dev, dt, m, n, k):
    """Q4_K / Q6_K from 128 rows with short rows: the wide-tile kernels (Q4_K
    in 32 x 64 tiles for the first three grids and 64 x 128 for the fourth,
    Q6_K in 64 x 128; one to five superblocks through the two-slot LDS ring,
    a ragged last row tile and column tile), f32 and f16 outputs, against the
    oracle."""
    say("wide", dt, m, n, k)
    wq = weights(dt, n, k)
    x = acts(m, k)
    want = O.matmul(dt, x, wq)
    out = dev.alloc((m, n), np.float32)
    F.qmatmul_f32_rocm_wrapper([dev.from_numpy(x), dev.from_numpy(as_u32(wq))], [out],
                               F.QMatMulParams(dt, 1, m, n, k))
    err = rel_err(out.numpy(), want)
    say("  rel_err", err)
    assert err <= TOL
    qs = dev.load_quantized(dt, wq.tobytes())
    x16 = O.f32_to_f16_bits(x)
    y16, _ = qs.fwd((n, k), dev.from_numpy(x16.view(np.float16)))
    err16 = rel_err(O.f16_bits_to_f32(y16.numpy().view(np.uint16)), O.f16_bits_to_f32(O.matmul_f16(dt, x16, wq)))
    say("  f16 rel_err", err16)
    assert err16 <= TOL_F16


@pytest.mark.parametrize("m", [64, 128])
def test_qmatmul_q4k_weights_off_16_byte_alignment(dev, m):
    """Q4_K blocks at a 4-byte (not 16-byte) aligned address, as a KernelRef
    input slice may be: the LDS-DMA staging needs 16-byte aligned blocks, so
    the plan takes the register-staged kernel; same results."""
    k, n = 2048, 320
    wq = weights(O.Q4K, n, k)
    x = acts(m, k)
    want = O.matmul(O.Q4K, x, wq)
    raw = as_u32(wq)
    buf = dev.from_numpy(np.concatenate([np.zeros(1, np.uint32), raw]))
    import ctypes as C
    from fuel_amd._native import check, lib
    xd = dev.from_numpy(x)
    out = dev.alloc((m, n), np.float32)
    check(lib().frq_qmatmul(dev.handle, O.Q4K, 1, m, n, k, C.c_void_p(xd.ptr), x.nbytes, C.c_void_p(buf.ptr + 4),
                            raw.nbytes, C.c_void_p(out.ptr), out.nbytes))
    err = rel_err(out.numpy(), want)
    say("  misaligned q4k m", m, "rel_err", err)
    assert err <= TOL


def test_qmatmul_workspace_holds_only_the_split_it_uses():
    """A QMatMul whose tiles fill the GPU runs unsplit and sizes its workspace
    for the quantized rows alone (no split-K partials): M = 1024 rows,
    N = 32000, K = 4096 would otherwise reserve 16 * M * N floats (2.1 GB).
    On a handle of its own, so that no earlier call has grown the workspace."""
    import ctypes as C
    from fuel_amd._native import check, lib
    dev = F.RocmDevice(0)
    m, n, k = 1024, 32000, 4096
    wd = dev.alloc((n * (k // 256) * 144 // 4,), np.uint32)
    check(lib().frq_memset(dev.handle, C.c_void_p(wd.ptr), 0, wd.nbytes))
    xd = dev.alloc((m, k), np.float32)
    check(lib().frq_memset(dev.handle, C.c_void_p(xd.ptr), 0, xd.nbytes))
    out = dev.alloc((m, n), np.float32)
    check(lib().frq_qmatmul(dev.handle, O.Q4K, 1, m, n, k, C.c_void_p(xd.ptr), xd.nbytes, C.c_void_p(wd.ptr),
                            wd.nbytes, C.c_void_p(out.ptr), out.nbytes))
    dev.synchronize()
    ws = C.c_size_t()
    check(lib().frq_device_workspace_bytes(dev.handle, C.byref(ws)))
    act = m * k + m * (k // 256) * 4 + m * (k // 256) * 32   # Q8K rows: qs, d, bsums
    say("  workspace bytes", ws.value, "quantized rows", act)
    assert ws.value < 2 * act + (1 << 20)
    assert np.all(out.numpy() == 0)
    del wd, xd, out
    dev.close()


@pytest.mark.parametrize("dt", [O.Q4K, O.Q6K])
@pytest.mark.parametrize("batch,m,n,k", [(1, 40, 100, 512), (3, 17, 130, 768), (1, 200, 70, 256)])
def test_qmatmul_mfma_ragged(dev, dt, batch, m, n, k):
    # row and column tails that do not fill a tile; the last Q6_K block of the
    # weights ends the allocation (its 2-byte-aligned tail chunk stays inside)
    say("mfma ragged", dt, batch, m, n, k)
    wq = weights(dt, n, k)
    assert wq.nbytes % 4 == 0  # fuel's U32 weight storage: these shapes give whole words
    x = acts(batch * m, k)
    want = O.matmul(dt, x, wq)
    out = dev.alloc((batch, m, n), np.float32)
    F.qmatmul_f32_rocm_wrapper([dev.from_numpy(x.reshape(batch, m, k)), dev.from_numpy(as_u32(wq))], [out],
                               F.QMatMulParams(dt, batch, m, n, k))
    assert rel_err(out.numpy().reshape(batch * m, n), want) <= TOL


def test_qmatmul_q6k_mfma_extreme_scales(dev):
    """Q6_K blocks at the ends of the code and scale ranges (codes 0 and 63,
    scales -128 and 127) against the exact integer sum: the 7-bit plane split
    of (q - 32) * sc must carry the full [-4096, 4064] product range."""
    say("mfma q6k extremes")
    m, n, k = 32, 64, 512
    rng = np.random.default_rng(5)
    blocks = np.zeros((n, k // 256), dtype=O.BLOCK_DTYPE[O.Q6K])
    raw = blocks.view(np.uint8).reshape(n, k // 256, 210)
    raw[..., :192] = rng.choice(np.array([0x00, 0xff, 0xf0, 0x0f], np.uint8), size=raw[..., :192].shape)
    raw[..., 192:208] = rng.choice(np.array([0x80, 0x7f, 0x01, 0xff], np.uint8), size=raw[..., 192:208].shape)
    raw[..., 208:210] = np.frombuffer(np.float16(1.0 / 4096).tobytes(), np.uint8)
    x = acts(m, k)
    want = O.matmul(O.Q6K, x, blocks)
    out = dev.alloc((m, n), np.float32)
    F.qmatmul_f32_rocm_wrapper([dev.from_numpy(x), dev.from_numpy(as_u32(blocks))], [out],
                               F.QMatMulParams(O.Q6K, 1, m, n, k))
    err = rel_err(out.numpy(), want)
    say("  rel_err", err)
    assert err <= TOL


def test_storage_outlives_device_close(dev):
    """A quantized storage freed after its device handle was closed releases
    cleanly, and the next calls on another handle see no error of it."""
    say("storage outlives close")
    d2 = F.RocmDevice(0)
    q = d2.qzeros(256 * 64, F.Q4K)
    d2.close()
    del q                                    # frees the blocks through the closed handle's record
    w = O.quantize(O.Q4K, O.normal((64, 256), seed=5, stream=1, std=0.02))
    x = O.normal((1, 256), seed=5, stream=2)
    got, _ = dev.load_quantized(O.Q4K, w.tobytes()).fwd((64, 256), dev.from_numpy(x))
    assert rel_err(got.numpy()[0], O.matmul(O.Q4K, x, w)[0]) < TOL


# ---- the quantize inside the mat-vec, bit for bit ----

def one_hot_q4k(k):
    """Q4_K weights [k, k/256]: row n is 1.0 at element n and 0 elsewhere (d =
    1, dmin = 0, every 6-bit scale 1, min 0), so y[n] = d_x * q8[n] of the
    activation's Q8K block, one f32 product."""
    kb = k // 256
    b = np.zeros((k, kb), O.BLOCK_Q4K)
    b["d"] = 0x3C00
    b["scales"] = np.array([1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1], np.uint8)
    n = np.arange(k)
    e = n % 256
    c, i = e // 64, e % 64
    idx = 32 * c + (i % 32)
    qs = b["qs"]
    qs[n, n // 256, idx] = np.where(i < 32, 1, 16).astype(np.uint8)
    return b


def one_hot_q6k(k):
    """Q6_K weights [k, k/256]: row n is 1.0 at element n (d = 1, every scale
    1, code 33 there and 32 elsewhere)."""
    kb = k // 256
    b = np.zeros((k, kb), O.BLOCK_Q6K)
    b["d"] = 0x3C00
    b["scales"] = 1
    b["qh"] = 0xAA  # the high two bits of code 32 (and 33) in every slot
    n = np.arange(k)
    e = n % 256
    hh, r = e // 128, e % 128
    qd, l = r // 32, r % 32
    ql = b["ql"]
    ql[n, n // 256, 64 * hh + l + 32 * (qd & 1)] = np.where(qd >> 1, 16, 1).astype(np.uint8)
    return b


@pytest.mark.parametrize("dt", [O.Q4K, O.Q6K])
@pytest.mark.parametrize("k", [256, 4096, 11008, 12288])
def test_matvec_fused_quantize_bit_exact(dev, dt, k):
    """The Q8K quantize the mat-vec runs on its activation row inside each
    workgroup (BlockQ8K::from_float, k_quants.rs:2230-2267), bit for bit:
    against one-hot weights every output is d_x * q8 of one element, which
    must equal the same product of the CPU path's Q8K block.  Rows: N(0, 1),
    the integer closed form, first-index ties, a zero row, and 2 rows (the
    several-row mat-vec)."""
    w = one_hot_q4k(k) if dt == O.Q4K else one_hot_q6k(k)
    rows = np.concatenate([acts(2, k, seed=k), special_rows(k)])
    wd = dev.from_numpy(as_u32(w))
    say("fused quantize", dt, k, rows.shape)
    for m in (1, 2):
        for r0 in range(0, rows.shape[0], m):
            x = rows[r0:r0 + m]
            if x.shape[0] < m:
                continue
            blk = O.quantize(O.Q8K, x)
            # (+ 0: the sums start from +0, so a zero product of a negative d is +0)
            want = (blk["d"][:, :, None] * blk["qs"].astype(np.float32)).reshape(m, k).astype(np.float32) + np.float32(0)
            out = dev.alloc((m, k), np.float32)
            F.qmatmul_f32_rocm_wrapper([dev.from_numpy(x), wd], [out], F.QMatMulParams(dt, 1, m, k, k))
            got = out.numpy()
            bad = np.nonzero(got.view(np.uint32) != want.view(np.uint32))
            assert bad[0].size == 0, (m, r0, bad[1][:8], got[bad][:8], want[bad][:8])
