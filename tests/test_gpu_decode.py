"""GPU parity of the decode-step path (fused mat-vecs, decode attention,
greedy step, the LLaMA-shaped decoder) against the CPU oracle, through the C ABI.

Bit-exact: the rotated, f16-rounded cache rows the attention kernel appends
(rope_f32 byte_kernels.rs:1885-1964 has no fused multiply-add; neither has the
kernel), the greedy token (argmax_dim_f32, first index on ties).  f32: the
fused QMatMuls within 1e-3 of the CPU output norm;
attention within 1e-5 (f32 only, no quantization).  Decoder logits: within
1e-2 of their norm.  GPU and CPU agree to ~1e-8 until an f32 ordering
difference of that size flips one Q8K activation rounding or one f16
KV-cache rounding; a flipped cache row then persists and the logits settle
near 3e-3 (measured over 20 steps of the small model).  Planted mistakes in
the decoder (rotation sign, score scale, norm gain, gate/up swap) move the
logits by 2.7e-2 .. 9.6e-2.
"""
import ctypes as C

import numpy as np
import pytest

import fuel_amd as F
import oracle as O
from blockref import rel_err
from fuel_amd.hiprt import HipRuntime
from fuel_amd.llama import LlamaConfig, LlamaDecoder
from oracle.llama import LlamaConfig as OConfig, OracleLlama

pytestmark = pytest.mark.gpu

TOL = 1e-3
DEC_TOL = 1e-2
L = F.lib


def say(*a):
    print(*a, flush=True)


def fused(dev, dt, w, x, n, k, m=1, ldx=None, x2=None, gain=None, eps=1e-5, acc=0, y=None, ldy=None, x_off=0):
    ldx = ldx or k
    ldy = ldy or n
    if y is None:
        y = dev.alloc((m, ldy), np.float32)
    F._native.check(L().frq_qmatmul_fused(dev.handle, dt, m, n, k, C.c_void_p(w.ptr), C.c_void_p(x.ptr + 4 * x_off), ldx,
                                          C.c_void_p(x2) if x2 else None, C.c_void_p(gain.ptr) if gain else None,
                                          eps, acc, C.c_void_p(y.ptr), ldy))
    return y


@pytest.mark.parametrize("dt,n,k,m", [(O.Q4K, 8192, 4096, 1), (O.Q6K, 4096, 4096, 1), (O.Q4K, 1000, 1024, 3),
                                      (O.Q8_0, 512, 2048, 2), (O.Q6K, 32000, 4096, 1)])
def test_qmatmul_fused_rms_norm(dev, dt, n, k, m):
    say("fused rms", dt, n, k, m)
    w = O.quantize(dt, O.normal((n, k), seed=n + k, stream=1, std=0.02))
    x = O.normal((m, k), seed=n + k, stream=2, std=3.0)
    g = 1 + O.normal((k,), seed=n + k, stream=3, std=0.2)
    wd, xd, gd = dev.from_numpy(w.view(np.uint8)), dev.from_numpy(x), dev.from_numpy(g)
    got = fused(dev, dt, wd, xd, n, k, m=m, gain=gd).numpy()
    want = O.matmul(dt, O.rms_norm(x, g, 1e-5), w)
    for r in range(m):
        assert rel_err(got[r], want[r]) < TOL, r


@pytest.mark.parametrize("dt,n,ffn", [(O.Q4K, 4096, 11008), (O.Q6K, 4096, 11008), (O.Q4K, 300, 512)])
def test_qmatmul_fused_swiglu_residual(dev, dt, n, ffn):
    say("fused swiglu", dt, n, ffn)
    w = O.quantize(dt, O.normal((n, ffn), seed=ffn, stream=1, std=0.02))
    gu = O.normal((2 * ffn,), seed=ffn, stream=2, std=2.0)
    y0 = O.normal((n,), seed=ffn, stream=3)
    wd, gud, y = dev.from_numpy(w.view(np.uint8)), dev.from_numpy(gu), dev.from_numpy(y0)
    fused(dev, dt, wd, gud, n, ffn, x2=gud.ptr + 4 * ffn, acc=1, y=y)
    g, u = gu[:ffn], gu[ffn:]
    h = (g / (np.float32(1) + np.exp(-g)) * u).astype(np.float32)
    want = y0 + O.matmul(dt, h[None], w)[0]
    assert rel_err(y.numpy(), want) < TOL


@pytest.mark.parametrize("dt,n,k,m,rms", [(O.Q4K, 11008, 4096, 1, True), (O.Q6K, 1000, 2048, 2, True),
                                          (O.Q8_0, 300, 1024, 3, False), (O.Q4K, 513, 4096, 1, False),
                                          (O.Q4K, 270000, 256, 1, True)])
def test_qmatmul_fused_glu(dev, dt, n, k, m, rms):
    """silu(gate . a) * (up . a) in one launch: the gate and up sums are the
    fused mat-vec's own (bit-identical), the product is silu_mul's; and the
    CPU path (QMatMul gate and up, SiLU·mul) within 1e-3 of its norm.  (270000
    rows: more than 64 a wavefront, which the launcher splits over launches.)"""
    say("fused glu", dt, n, k, m, rms)
    wg = O.quantize(dt, O.normal((n, k), seed=n + k, stream=1, std=0.02))
    wu = O.quantize(dt, O.normal((n, k), seed=n + k, stream=2, std=0.02))
    x = O.normal((m, k), seed=n + k, stream=3, std=2.0)
    g = 1 + O.normal((k,), seed=n + k, stream=4, std=0.2)
    wgd, wud, xd, gd = (dev.from_numpy(a) for a in (wg.view(np.uint8), wu.view(np.uint8), x, g))
    y = dev.alloc((m, n), np.float32)
    F._native.check(L().frq_qmatmul_fused_glu(dev.handle, dt, m, n, k, C.c_void_p(wgd.ptr), C.c_void_p(wud.ptr),
                                              C.c_void_p(xd.ptr), k, C.c_void_p(gd.ptr) if rms else None, 1e-5,
                                              C.c_void_p(y.ptr), n))
    got = y.numpy()
    # (row by row: the one-row fused launch is the mat-vec the GLU mode extends;
    # several rows take the batched MFMA path, whose f32 sums differ in order)
    sg = np.concatenate([fused(dev, dt, wgd, xd, n, k, m=1, gain=gd if rms else None, x_off=r * k).numpy()
                         for r in range(m)])
    su = np.concatenate([fused(dev, dt, wud, xd, n, k, m=1, gain=gd if rms else None, x_off=r * k).numpy()
                         for r in range(m)])
    host = (sg / (np.float32(1) + np.exp(-sg)) * su).astype(np.float32)
    np.testing.assert_allclose(got, host, rtol=2e-6, atol=0)  # (device expf vs numpy exp: an ulp or two)
    xn = O.rms_norm(x, g, 1e-5) if rms else x
    gw, uw = O.matmul(dt, xn, wg), O.matmul(dt, xn, wu)
    want = (gw / (np.float32(1) + np.exp(-gw)) * uw).astype(np.float32)
    for r in range(m):
        assert rel_err(got[r], want[r]) < TOL, r


@pytest.mark.parametrize("dt,n,k,m,mode", [
    (O.Q4K, 8192, 4096, 2, "rms"), (O.Q6K, 4096, 4096, 17, "rms"), (O.Q4K, 8192, 4096, 128, "rms"),
    (O.Q6K, 1000, 4096, 33, "rms"), (O.Q4K, 22016, 4096, 512, "rms"),
    (O.Q4K, 4096, 11008, 3, "swiglu"), (O.Q6K, 4096, 11008, 64, "swiglu"), (O.Q4K, 4096, 11008, 512, "swiglu"),
    (O.Q6K, 4096, 4096, 40, "plain"), (O.Q4K, 4096, 4096, 512, "plain"), (O.Q4K, 700, 2048, 5, "plain"),
    (O.Q4K, 22016, 4096, 8, "rms"), (O.Q4K, 4096, 11008, 24, "swiglu"), (O.Q6K, 32000, 4096, 8, "rms")])
def test_qmatmul_fused_batched(dev, dt, n, k, m, mode):
    """Several rows through the fused entry point (the batched prompt pass):
    the rows formed by the prologue (RMS norm x gain, the SwiGLU product of
    strided g | u rows, or strided plain rows), quantized once, the int8-MFMA
    kernels with the residual added in their epilogue -- within 1e-3 of the
    CPU path (quantize, matmul, then the residual add) row by row."""
    say("fused batched", dt, n, k, m, mode)
    w = O.quantize(dt, O.normal((n, k), seed=n + k + m, stream=1, std=0.02))
    wd = dev.from_numpy(w.view(np.uint8))
    ldx = 2 * k if mode != "rms" else k + 256  # strided rows
    xs = O.normal((m, ldx), seed=n + k + m, stream=2, std=2.0)
    xd = dev.from_numpy(xs)
    y0 = O.normal((m, n), seed=n + k + m, stream=3)
    if mode == "rms":
        g = 1 + O.normal((k,), seed=n + k, stream=4, std=0.2)
        gd = dev.from_numpy(g)
        got = fused(dev, dt, wd, xd, n, k, m=m, ldx=ldx, gain=gd).numpy()
        want = O.matmul(dt, O.rms_norm(np.ascontiguousarray(xs[:, :k]), g, 1e-5), w)
    elif mode == "swiglu":
        yd = dev.from_numpy(y0)
        got = fused(dev, dt, wd, xd, n, k, m=m, ldx=ldx, x2=xd.ptr + 4 * k, acc=1, y=yd).numpy()
        gg, uu = xs[:, :k], xs[:, k:]
        h = (gg / (np.float32(1) + np.exp(-gg)) * uu).astype(np.float32)
        want = y0 + O.matmul(dt, h, w)
    else:
        yd = dev.from_numpy(y0)
        got = fused(dev, dt, wd, xd, n, k, m=m, ldx=ldx, acc=1, y=yd).numpy()
        want = y0 + O.matmul(dt, np.ascontiguousarray(xs[:, :k]), w)
    for r in range(m):
        assert rel_err(got[r], want[r]) < TOL, r


@pytest.mark.parametrize("dt,n,k,m", [(O.Q4K, 4096, 4096, 512), (O.Q6K, 4096, 4096, 16), (O.Q4K, 1000, 2048, 40)])
def test_qmatmul_fused_batched_plain_matches_qmatmul(dev, dt, n, k, m):
    """Contiguous plain rows through the fused entry point run frq_qmatmul's own
    quantize and kernels: without accumulate the outputs are bit-identical, with
    it they are the f32 sum y0 + those outputs."""
    say("fused batched plain", dt, n, k, m)
    w = O.quantize(dt, O.normal((n, k), seed=n + k, stream=5, std=0.02))
    x = O.normal((m, k), seed=n + k, stream=6)
    y0 = O.normal((m, n), seed=n + k, stream=7)
    wd, xd = dev.from_numpy(w.view(np.uint8)), dev.from_numpy(x)
    ref = dev.alloc((m, n), np.float32)
    F.qmatmul_f32_rocm_wrapper([xd, dev.from_numpy(np.frombuffer(w.tobytes(), np.uint32))], [ref],
                               F.QMatMulParams(dt, 1, m, n, k))
    ref = ref.numpy()
    np.testing.assert_array_equal(fused(dev, dt, wd, xd, n, k, m=m).numpy(), ref)
    yd = dev.from_numpy(y0)
    np.testing.assert_array_equal(fused(dev, dt, wd, xd, n, k, m=m, acc=1, y=yd).numpy(), (y0 + ref).astype(np.float32))


@pytest.mark.parametrize("dt1,n1,dt2,n2,k,m", [(O.Q4K, 8192, O.Q6K, 4096, 4096, 1), (O.Q6K, 300, O.Q4K, 1000, 2048, 2),
                                               (O.Q4K, 512, O.Q4K, 768, 11008, 1), (O.Q4K, 8192, O.Q6K, 4096, 4096, 48),
                                               (O.Q4K, 8192, O.Q6K, 4096, 4096, 512)])
def test_qmatmul_fused_pair(dev, dt1, n1, dt2, n2, k, m):
    """[q|k] and v from one launch equal the two single fused launches (same
    kernels, same quantized activation) and the CPU path within 1e-3."""
    say("fused pair", dt1, n1, dt2, n2, k, m)
    w1 = O.quantize(dt1, O.normal((n1, k), seed=k, stream=1, std=0.02))
    w2 = O.quantize(dt2, O.normal((n2, k), seed=k, stream=2, std=0.02))
    x = O.normal((m, k), seed=k, stream=3, std=2.0)
    g = 1 + O.normal((k,), seed=k, stream=4, std=0.2)
    w1d, w2d, xd, gd = (dev.from_numpy(a) for a in (w1.view(np.uint8), w2.view(np.uint8), x, g))
    y1, y2 = dev.alloc((m, n1), np.float32), dev.alloc((m, n2), np.float32)
    F._native.check(L().frq_qmatmul_fused_pair(dev.handle, m, k, C.c_void_p(xd.ptr), k, C.c_void_p(gd.ptr), 1e-5,
                                               dt1, n1, C.c_void_p(w1d.ptr), C.c_void_p(y1.ptr),
                                               dt2, n2, C.c_void_p(w2d.ptr), C.c_void_p(y2.ptr)))
    s1 = fused(dev, dt1, w1d, xd, n1, k, m=m, gain=gd).numpy()
    s2 = fused(dev, dt2, w2d, xd, n2, k, m=m, gain=gd).numpy()
    np.testing.assert_array_equal(y1.numpy(), s1)
    np.testing.assert_array_equal(y2.numpy(), s2)
    xn = O.rms_norm(x, g, 1e-5)
    w1r, w2r = O.matmul(dt1, xn, w1), O.matmul(dt2, xn, w2)
    for r in range(m):
        assert rel_err(y1.numpy()[r], w1r[r]) < TOL and rel_err(y2.numpy()[r], w2r[r]) < TOL


def test_qmatmul_fused_errors(dev):
    w = dev.alloc((144 * 16,), np.uint8)
    x = dev.alloc((4096,), np.float32)
    g = dev.alloc((4096,), np.float32)
    with pytest.raises(F.FuelRocmError):  # rms gain and swiglu together
        fused(dev, O.Q4K, w, x, 1, 4096, x2=x.ptr, gain=g)
    with pytest.raises(F.FuelRocmError):  # k not a block multiple
        fused(dev, O.Q4K, w, x, 1, 100)
    with pytest.raises(F.FuelRocmError):  # misaligned x
        F._native.check(L().frq_qmatmul_fused(dev.handle, O.Q4K, 1, 1, 256, C.c_void_p(w.ptr),
                                              C.c_void_p(x.ptr + 4), 256, None, None, 0.0, 0,
                                              C.c_void_p(x.ptr), 1))


# ---- decode attention ----

class Attn:
    def __init__(self, dev, H, max_ctx):
        self.dev, self.H, self.C = dev, H, max_ctx
        self.kc = dev.alloc((H, max_ctx, 128), np.uint16)
        self.vc = dev.alloc((H, max_ctx, 128), np.uint16)
        self.wb = int(L().frq_attention_decode_workspace(H, max_ctx))
        self.work = dev.alloc((self.wb,), np.uint8)
        self.work.copy_from(np.zeros(self.wb, np.uint8))
        c, s = O.rope_tables(10000.0, 0, max_ctx, 128)
        self.cos, self.sin = c, s
        self.cd, self.sd = dev.from_numpy(c), dev.from_numpy(s)
        self.out = dev.alloc((H, 128), np.float32)
        self.posd = dev.alloc((1,), np.int32)

    def run(self, qk, v, pos):
        self.posd.copy_from(np.array([pos], np.int32))
        qkd, vd = self.dev.from_numpy(qk), self.dev.from_numpy(v)
        F._native.check(L().frq_attention_decode(
            self.dev.handle, self.H, 128, self.C, C.c_void_p(qkd.ptr), C.c_void_p(vd.ptr), C.c_void_p(self.cd.ptr),
            C.c_void_p(self.sd.ptr), C.c_void_p(self.kc.ptr), C.c_void_p(self.vc.ptr), C.c_void_p(self.posd.ptr),
            float(np.float32(1 / np.sqrt(128.0))), C.c_void_p(self.work.ptr), self.wb, C.c_void_p(self.out.ptr)))
        return self.out.numpy()


@pytest.mark.parametrize("H,max_ctx,pos", [(4, 64, 0), (4, 64, 1), (4, 64, 37), (4, 64, 63), (32, 768, 700),
                                           (3, 2048, 1500)])
def test_attention_decode(dev, H, max_ctx, pos):
    say("attention", H, max_ctx, pos)
    a = Attn(dev, H, max_ctx)
    rng = np.random.default_rng(pos + H)
    kc = rng.standard_normal((H, max_ctx, 128)).astype(np.float16)
    vc = rng.standard_normal((H, max_ctx, 128)).astype(np.float16)
    # rows pos.. are not attended (row pos is replaced by the append): NaN there
    # must not reach the output
    kc[:, pos:] = np.float16(np.nan)
    vc[:, pos:] = np.float16(np.nan)
    a.kc.copy_from(kc.view(np.uint16))
    a.vc.copy_from(vc.view(np.uint16))
    qk = O.normal((2 * H * 128,), seed=pos, stream=1, std=2.0)
    v = O.normal((H * 128,), seed=pos, stream=2)
    got = a.run(qk, v, pos)
    # the appended rows: rope'd k and v rounded to f16, bit-exact
    q = O.rope(qk[:H * 128].reshape(H, 1, 128), a.cos[pos:pos + 1], a.sin[pos:pos + 1]).reshape(H, 128)
    k = O.rope(qk[H * 128:].reshape(H, 1, 128), a.cos[pos:pos + 1], a.sin[pos:pos + 1]).reshape(H, 128)
    kc[:, pos] = k.astype(np.float16)
    vc[:, pos] = v.reshape(H, 128).astype(np.float16)
    np.testing.assert_array_equal(a.kc.numpy()[:, pos], kc[:, pos].view(np.uint16))
    np.testing.assert_array_equal(a.vc.numpy()[:, pos], vc[:, pos].view(np.uint16))
    kc[:, pos + 1:] = 0
    vc[:, pos + 1:] = 0
    want = O.attention_decode(q, kc.astype(np.float32), vc.astype(np.float32), pos + 1,
                              float(np.float32(1 / np.sqrt(128.0))))
    assert rel_err(got, want) < 1e-5
    # the workspace is reusable: a second call gives the same result
    np.testing.assert_array_equal(a.run(qk, v, pos), got)


def test_attention_decode_sequence(dev):
    """64 consecutive steps (positions 600..663, 32 heads, fresh q, k, v each
    step) reusing one workspace: every step's output within 1e-5 of the CPU
    attention over the cache as it stands, every appended row bit-exact.  A
    merge that read a split partial left by the previous step (another q)
    would miss by far more."""
    H, max_ctx = 32, 768
    a = Attn(dev, H, max_ctx)
    rng = np.random.default_rng(5)
    kc = rng.standard_normal((H, max_ctx, 128)).astype(np.float16)
    vc = rng.standard_normal((H, max_ctx, 128)).astype(np.float16)
    a.kc.copy_from(kc.view(np.uint16))
    a.vc.copy_from(vc.view(np.uint16))
    scale = float(np.float32(1 / np.sqrt(128.0)))
    for pos in range(600, 664):
        qk = O.normal((2 * H * 128,), seed=pos, stream=11, std=2.0)
        v = O.normal((H * 128,), seed=pos, stream=12)
        got = a.run(qk, v, pos)
        q = O.rope(qk[:H * 128].reshape(H, 1, 128), a.cos[pos:pos + 1], a.sin[pos:pos + 1]).reshape(H, 128)
        k = O.rope(qk[H * 128:].reshape(H, 1, 128), a.cos[pos:pos + 1], a.sin[pos:pos + 1]).reshape(H, 128)
        kc[:, pos] = k.astype(np.float16)
        vc[:, pos] = v.reshape(H, 128).astype(np.float16)
        want = O.attention_decode(q, kc[:, :pos + 1].astype(np.float32), vc[:, :pos + 1].astype(np.float32), pos + 1,
                                  scale)
        assert rel_err(got, want) < 1e-5, pos
    np.testing.assert_array_equal(a.kc.numpy()[:, 600:664], kc[:, 600:664].view(np.uint16))
    np.testing.assert_array_equal(a.vc.numpy()[:, 600:664], vc[:, 600:664].view(np.uint16))


@pytest.mark.parametrize("H,max_ctx,pos,dt,n", [(32, 768, 700, O.Q4K, 4096), (32, 1024, 0, O.Q6K, 4096),
                                                 (32, 768, 768, O.Q4K, 4096), (2, 64, 0, O.Q6K, 300),
                                                 (2, 2048, 1500, O.Q8_0, 512), (4, 1024, 1023, O.Q4K, 1000),
                                                 (2, 64, 64, O.Q4K, 256), (64, 512, 300, O.Q4K, 1000),
                                                 (128, 256, 100, O.Q6K, 512)])
def test_attention_decode_oproj(dev, H, max_ctx, pos, dt, n):
    """Attention + o-projection + residual equals frq_attention_decode then
    the fused QMatMul with accumulate, bit for bit (same caches, appends and
    outputs): 8, 4 and 2 splits (32, 64 and 128 heads: the merge inside the
    mat-vec, two launches), 64 and 128 splits (the merge kernel into the
    workspace tail), and an out-of-range pos (NaN attention, no append) on
    both paths."""
    say("attention oproj", H, max_ctx, pos, dt, n)
    k = H * 128
    rng = np.random.default_rng(pos + H)
    kc0 = rng.standard_normal((H, max_ctx, 128)).astype(np.float16)
    vc0 = rng.standard_normal((H, max_ctx, 128)).astype(np.float16)
    qk = O.normal((2 * k,), seed=pos, stream=1, std=2.0)
    v = O.normal((k,), seed=pos, stream=2)
    w = O.quantize(dt, O.normal((n, k), seed=n, stream=3, std=0.02))
    y0 = O.normal((n,), seed=n, stream=4)
    wd = dev.from_numpy(w.view(np.uint8))
    scale = float(np.float32(1 / np.sqrt(128.0)))
    outs = []
    for fused_path in (False, True):
        a = Attn(dev, H, max_ctx)
        a.kc.copy_from(kc0.view(np.uint16))
        a.vc.copy_from(vc0.view(np.uint16))
        a.posd.copy_from(np.array([pos], np.int32))
        qkd, vd, y = dev.from_numpy(qk), dev.from_numpy(v), dev.from_numpy(y0)
        args = (dev.handle, H, 128, max_ctx, C.c_void_p(qkd.ptr), C.c_void_p(vd.ptr), C.c_void_p(a.cd.ptr),
                C.c_void_p(a.sd.ptr), C.c_void_p(a.kc.ptr), C.c_void_p(a.vc.ptr), C.c_void_p(a.posd.ptr), scale,
                C.c_void_p(a.work.ptr), a.wb)
        if fused_path:
            F._native.check(L().frq_attention_decode_oproj(*args, dt, C.c_void_p(wd.ptr), n, C.c_void_p(y.ptr)))
        else:
            F._native.check(L().frq_attention_decode(*args, C.c_void_p(a.out.ptr)))
            fused(dev, dt, wd, a.out, n, k, acc=1, y=y)
        outs.append((y.numpy(), a.kc.numpy(), a.vc.numpy()))
    (y_ref, kc_ref, vc_ref), (y_got, kc_got, vc_got) = outs
    np.testing.assert_array_equal(kc_got, kc_ref)
    np.testing.assert_array_equal(vc_got, vc_ref)
    np.testing.assert_array_equal(y_got, y_ref)  # (NaN == NaN here)
    if pos < max_ctx:
        assert np.isfinite(y_got).all()


def test_attention_decode_oproj_errors(dev):
    a = Attn(dev, 2, 64)
    w = dev.alloc((256 * 144,), np.uint8)
    y = dev.alloc((256,), np.float32)
    base = (dev.handle, 2, 128, 64, C.c_void_p(y.ptr), C.c_void_p(y.ptr), C.c_void_p(a.cd.ptr), C.c_void_p(a.sd.ptr),
            C.c_void_p(a.kc.ptr), C.c_void_p(a.vc.ptr), C.c_void_p(a.posd.ptr), 0.1)
    with pytest.raises(F.FuelRocmError):  # workspace too small
        F._native.check(L().frq_attention_decode_oproj(*base, C.c_void_p(a.work.ptr), a.wb - 4, O.Q4K,
                                                       C.c_void_p(w.ptr), 256, C.c_void_p(y.ptr)))
    with pytest.raises(F.FuelRocmError):  # workspace not 16-byte aligned
        F._native.check(L().frq_attention_decode_oproj(*base, C.c_void_p(a.work.ptr + 4), a.wb, O.Q4K,
                                                       C.c_void_p(w.ptr), 256, C.c_void_p(y.ptr)))
    with pytest.raises(F.FuelRocmError):  # not a weight type
        F._native.check(L().frq_attention_decode_oproj(*base, C.c_void_p(a.work.ptr), a.wb, 0,
                                                       C.c_void_p(w.ptr), 256, C.c_void_p(y.ptr)))
    with pytest.raises(F.FuelRocmError):  # n_heads * head_dim not a multiple of 256
        F._native.check(L().frq_attention_decode_oproj(dev.handle, 1, 128, 64, *base[4:], C.c_void_p(a.work.ptr),
                                                       a.wb, O.Q4K, C.c_void_p(w.ptr), 256, C.c_void_p(y.ptr)))


def test_attention_decode_pos_out_of_range(dev):
    a = Attn(dev, 2, 16)
    a.kc.copy_from(np.zeros((2, 16, 128), np.uint16))
    got = a.run(O.normal((512,), seed=1, stream=1), O.normal((256,), seed=1, stream=2), 16)
    assert np.isnan(got).all()
    assert (a.kc.numpy() == 0).all()


# ---- greedy step ----

def test_argmax_embed(dev):
    vocab, dim, cap = 1000, 64, 16
    table = O.normal((vocab, dim), seed=3, stream=1)
    logits = O.normal((vocab,), seed=3, stream=2)
    logits[[17, 400, 999]] = logits.max() + 1          # tie: the first index wins
    td, ld = dev.from_numpy(table), dev.from_numpy(logits)
    toks = dev.from_numpy(np.array([5, 9, 11] + [0] * (cap - 3), np.int32))
    pos = dev.from_numpy(np.array([0], np.int32))
    x = dev.alloc((dim,), np.float32)

    plen = dev.alloc((1,), np.int32)

    def step(prompt_len):
        plen.copy_from(np.array([prompt_len], np.int32))
        F._native.check(L().frq_argmax_embed(dev.handle, C.c_void_p(ld.ptr), vocab, C.c_void_p(td.ptr), dim,
                                             C.c_void_p(toks.ptr), cap, C.c_void_p(plen.ptr), C.c_void_p(pos.ptr),
                                             C.c_void_p(x.ptr)))

    step(3)   # pos 0 -> forced prompt token 9
    assert pos.numpy()[0] == 1 and toks.numpy()[1] == 9
    np.testing.assert_array_equal(x.numpy(), table[9])
    step(3)   # pos 1 -> forced 11
    np.testing.assert_array_equal(x.numpy(), table[11])
    step(3)   # pos 2 -> argmax
    assert toks.numpy()[3] == 17 == O.argmax(logits)
    np.testing.assert_array_equal(x.numpy(), table[17])
    assert pos.numpy()[0] == 3


# ---- the decoder ----

SMALL = dict(dim=256, n_layers=2, n_heads=2, head_dim=128, ffn=512, vocab=300, max_ctx=32)


def oracle_model(dec):
    wh = dec.weights_host()

    def blocks(t):
        raw, shape, dt = t
        return np.frombuffer(raw.tobytes(), dtype=O.BLOCK_DTYPE[dt]).reshape(shape)

    w = {"embed": wh["embed"], "final_gain": wh["final_gain"], "out": blocks(wh["out"]), "layers": []}
    for lw in wh["layers"]:
        w["layers"].append({k: (blocks(v) if isinstance(v, tuple) else v) for k, v in lw.items()})
    cfg = OConfig(**{k: getattr(dec.cfg, k) for k in SMALL}) if dec.cfg.dim == 256 else OConfig()
    return OracleLlama(cfg, w)


@pytest.fixture(scope="module")
def small_decoder(dev):
    return LlamaDecoder(dev, LlamaConfig(**SMALL), seed=99, std=0.05)


def test_decoder_teacher_forced_logits(dev, small_decoder):
    say("decoder teacher forced")
    dec = small_decoder
    ref = oracle_model(dec)
    prompt = [7, 123, 45, 299, 0, 18, 250, 3, 77, 140, 11, 5]
    dec.start(prompt)
    for p, t in enumerate(prompt):
        dec.enqueue_step()
        got = dec.logits.numpy()
        want = ref.step(t, p)
        err = rel_err(got, want)
        say("  pos", p, "rel_err", err)
        assert err < DEC_TOL, (p, err)
    # the caches hold the same rounded rows as the CPU path's
    kc, vc = dec.kv_host(1)
    assert rel_err(kc[:, :len(prompt)], ref.kc[1][:, :len(prompt)]) < DEC_TOL


def test_decoder_teacher_forced_layers(dev, small_decoder):
    """Per-layer parity at the north-star bound: after six forced steps, the
    seventh position layer by layer with the CPU path teacher-forced on the
    GPU's residual and caches (test_gpu_prefill.teacher_forced_layers)."""
    from test_gpu_prefill import teacher_forced_layers

    dec = small_decoder
    ref = oracle_model(dec)
    prompt = [7, 123, 45, 299, 0, 18, 250, 3]
    dec.start(prompt)
    for _ in range(6):
        dec.enqueue_step()
    assert dec.pos.numpy()[0] == 6
    teacher_forced_layers(dec, ref, 6)


def test_decoder_greedy_graph_replay(dev, small_decoder):
    """A captured step replays every position; tokens match the eager run's and
    the CPU path's greedy choices."""
    say("decoder graph replay")
    dec = small_decoder
    prompt = [1, 2, 3, 4, 5]
    n_steps = 20
    dec.start(prompt)
    for _ in range(n_steps):
        dec.enqueue_step()
    eager = dec.tokens_host()[:n_steps + 1].copy()
    hip = HipRuntime()
    s = hip.stream_create()
    dev.set_stream(s)
    try:
        dec.start(prompt)
        hip.stream_sync(s)
        g = hip.capture(s, dec.enqueue_step)
        dec.start(prompt)
        for _ in range(n_steps):
            hip.graph_launch(g, s)
        hip.stream_sync(s)
        replay = dec.tokens_host()[:n_steps + 1].copy()
        hip.graph_destroy(g)
    finally:
        dev.set_stream(None)
    np.testing.assert_array_equal(replay, eager)
    # Greedy parity under the logits tolerance: the CPU path, fed the GPU's
    # tokens, must rank every GPU pick first or within DEC_TOL of the logits'
    # norm of its own first choice (a near-tie that rounding may break either
    # way).
    ref = oracle_model(dec)
    toks = eager.tolist()
    exact = 0
    for p in range(n_steps):
        lg = ref.step(toks[p], p)
        if p + 1 >= len(prompt):
            best, chosen = ref.greedy(lg), toks[p + 1]
            gap = float(lg[best] - lg[chosen]) / float(np.linalg.norm(lg))
            say("  pos", p, "gpu", chosen, "cpu", best, "gap", gap)
            assert gap <= DEC_TOL, (p, chosen, best, gap)
            exact += chosen == best
    assert exact >= (n_steps - len(prompt) + 1) // 2


def test_decoder_graph_replays_another_prompt_length(dev, small_decoder):
    """The prompt length lives in device memory: a step captured while one
    prompt was loaded forces the tokens of a later, longer or shorter prompt
    exactly as the eager steps do."""
    say("decoder graph replay, other prompt lengths")
    dec = small_decoder
    hip = HipRuntime()
    s = hip.stream_create()
    dev.set_stream(s)
    try:
        dec.start([1, 2, 3])
        hip.stream_sync(s)
        g = hip.capture(s, dec.enqueue_step)
        for prompt in ([9, 8, 7, 6, 5, 4, 3], [42]):
            n_steps = 12
            dec.start(prompt)
            for _ in range(n_steps):
                dec.enqueue_step()
            eager = dec.tokens_host()[:n_steps + 1].copy()
            dec.start(prompt)
            for _ in range(n_steps):
                hip.graph_launch(g, s)
            hip.stream_sync(s)
            replay = dec.tokens_host()[:n_steps + 1].copy()
            assert replay[:len(prompt)].tolist() == prompt
            np.testing.assert_array_equal(replay, eager)
        hip.graph_destroy(g)
    finally:
        dev.set_stream(None)


def test_decoder_fused_oproj_matches_unfused(dev, small_decoder):
    """The decoder's attention-merging o-projection (five launches per layer)
    and its one-launch SwiGLU product give the same logits and tokens, bit for
    bit, as the separate merge kernel (six) and the SwiGLU product formed in
    the down projection's activation stage."""
    say("decoder fused oproj / glu")
    dec = small_decoder
    assert dec.fuse_oproj and dec.fuse_glu
    ref = LlamaDecoder(dev, LlamaConfig(**SMALL), seed=99, std=0.05, fuse_oproj=False, fuse_glu=False)
    assert ref.launches_per_step() == dec.launches_per_step() + SMALL["n_layers"]
    prompt = [3, 1, 4, 1, 5, 9, 2, 6]
    dec.start(prompt)
    ref.start(prompt)
    for _ in range(16):
        dec.enqueue_step()
        ref.enqueue_step()
        np.testing.assert_array_equal(dec.logits.numpy(), ref.logits.numpy())
    np.testing.assert_array_equal(dec.tokens_host()[:17], ref.tokens_host()[:17])


# ---- the decoder from a GGUF file ----

def write_gguf(path, dec, tied=False):
    """The decoder's weights as a GGUF file in llama.cpp's LLaMA layout."""
    from oracle import gguf as G

    cfg, wh = dec.cfg, dec.weights_host()
    md = [("general.architecture", G.Value(G.VT_STRING, "llama")),
          ("general.alignment", G.Value(G.VT_U32, 32)),
          ("llama.embedding_length", G.Value(G.VT_U32, cfg.dim)),
          ("llama.block_count", G.Value(G.VT_U32, cfg.n_layers)),
          ("llama.attention.head_count", G.Value(G.VT_U32, cfg.n_heads)),
          ("llama.attention.head_count_kv", G.Value(G.VT_U32, cfg.n_heads)),
          ("llama.feed_forward_length", G.Value(G.VT_U32, cfg.ffn)),
          ("llama.attention.layer_norm_rms_epsilon", G.Value(G.VT_F32, cfg.eps)),
          ("llama.rope.freq_base", G.Value(G.VT_F32, cfg.rope_theta))]
    d, f = cfg.dim, cfg.ffn

    def q(t, rows, cols):
        raw, _, dt = t
        return dt, (rows, cols), raw.tobytes()

    out_dt, _, out_raw = q(wh["out"], cfg.vocab, d)
    tens = []
    if tied:
        tens.append(("token_embd.weight", out_dt, (cfg.vocab, d), out_raw))
    else:
        tens.append(("token_embd.weight", 0, (cfg.vocab, d), wh["embed"].astype(np.float32).tobytes()))
        tens.append(("output.weight", out_dt, (cfg.vocab, d), out_raw))
    tens.append(("output_norm.weight", 0, (d,), wh["final_gain"].tobytes()))
    names = {"wq": "attn_q", "wk": "attn_k", "wv": "attn_v", "wo": "attn_output", "wg": "ffn_gate",
             "wu": "ffn_up", "wd": "ffn_down"}
    shape = {"wq": (d, d), "wk": (d, d), "wv": (d, d), "wo": (d, d), "wg": (f, d), "wu": (f, d), "wd": (d, f)}
    for li, lw in enumerate(wh["layers"]):
        for m, nm in names.items():
            dt, dims, raw = q(lw[m], *shape[m])
            tens.append((f"blk.{li}.{nm}.weight", dt, dims, raw))
        tens.append((f"blk.{li}.attn_norm.weight", 0, (d,), lw["attn_gain"].tobytes()))
        tens.append((f"blk.{li}.ffn_norm.weight", 1, (d,), lw["ffn_gain"].astype(np.float16).tobytes()))
    path.write_bytes(G.write(md, tens))


def test_decoder_from_gguf_matches(dev, small_decoder, tmp_path):
    """The same model read back from a GGUF file decodes bit-identically."""
    say("decoder from gguf")
    dec = small_decoder
    p = tmp_path / "small.gguf"
    write_gguf(p, dec)
    dec2 = LlamaDecoder.from_gguf(dev, str(p), max_ctx=dec.cfg.max_ctx)
    assert (dec2.cfg.dim, dec2.cfg.n_layers, dec2.cfg.n_heads, dec2.cfg.ffn, dec2.cfg.vocab) == \
        (dec.cfg.dim, dec.cfg.n_layers, dec.cfg.n_heads, dec.cfg.ffn, dec.cfg.vocab)
    prompt = [3, 141, 59, 26]
    runs = []
    for dd in (dec, dec2):
        dd.start(prompt)
        lg = []
        for _ in range(10):
            dd.enqueue_step()
            lg.append(dd.logits.numpy())
        runs.append((dd.tokens_host()[:11].copy(), np.stack(lg)))
    np.testing.assert_array_equal(runs[0][0], runs[1][0])
    assert np.array_equal(runs[0][1].view(np.uint32), runs[1][1].view(np.uint32))


def test_decoder_from_gguf_tied_output_and_errors(dev, small_decoder, tmp_path):
    """Without output.weight the quantized token_embd is the output matrix and
    the embedding table is its device dequantization (to_float)."""
    say("decoder from gguf, tied")
    dec = small_decoder
    p = tmp_path / "tied.gguf"
    write_gguf(p, dec, tied=True)
    dec3 = LlamaDecoder.from_gguf(dev, str(p), max_ctx=16)
    raw, shape, dt = dec.weights_host()["out"]
    blocks = np.frombuffer(raw.tobytes(), dtype=O.BLOCK_DTYPE[dt]).reshape(shape)
    np.testing.assert_array_equal(dec3.embed.numpy().view(np.uint32),
                                  O.dequantize(dt, blocks).reshape(dec.cfg.vocab, dec.cfg.dim).view(np.uint32))
    assert dec3.weights_host()["out"][0].tobytes() == raw.tobytes()
    from oracle import gguf as G
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(G.write([("general.architecture", G.Value(G.VT_STRING, "llama"))], []))
    with pytest.raises(ValueError, match="missing metadata|missing tensor"):
        LlamaDecoder.from_gguf(dev, str(bad))
