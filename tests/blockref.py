"""Element-wise decoders of the GGUF block formats, written from the format
definitions (to_float: k_quants.rs:611-627, 1595-1622, 2158-2189; Q8K
:2269-2280), used by tests as an independent brute-force check of the
oracle's and the GPU's blocked integer sums.  Test helper only."""
import numpy as np

import oracle as O


def q4k_fields(blocks: np.ndarray):
    """-> (d f32 [...], dmin f32 [...], sc int [...,8], mn int [...,8], q int [...,256])."""
    d = blocks["d"].view(np.float16).astype(np.float32)
    dmin = blocks["dmin"].view(np.float16).astype(np.float32)
    s = blocks["scales"].astype(np.int64)
    sc = np.empty(s.shape[:-1] + (8,), np.int64)
    mn = np.empty_like(sc)
    for j in range(8):
        if j < 4:
            sc[..., j] = s[..., j] & 63
            mn[..., j] = s[..., j + 4] & 63
        else:
            sc[..., j] = (s[..., j + 4] & 0xF) | ((s[..., j - 4] >> 6) << 4)
            mn[..., j] = (s[..., j + 4] >> 4) | ((s[..., j] >> 6) << 4)
    qs = blocks["qs"].astype(np.int64)
    e = np.arange(256)
    byte = qs[..., 32 * (e // 64) + e % 32]
    q = (byte >> (4 * ((e % 64) // 32))) & 0xF
    return d, dmin, sc, mn, q


def q6k_fields(blocks: np.ndarray):
    """-> (d f32 [...], sc int [...,16], q int [...,256] in [-32, 31])."""
    d = blocks["d"].view(np.float16).astype(np.float32)
    sc = blocks["scales"].astype(np.int64)
    ql = blocks["ql"].astype(np.int64)
    qh = blocks["qh"].astype(np.int64)
    e = np.arange(256)
    h, r = e // 128, e % 128
    qd, l = r // 32, r % 32
    lo = (ql[..., 64 * h + 32 * (qd % 2) + l] >> (4 * (qd // 2))) & 0xF
    hi = (qh[..., 32 * h + l] >> (2 * qd)) & 3
    return d, sc, (lo | (hi << 4)) - 32


def q8_0_fields(blocks: np.ndarray):
    return blocks["d"].view(np.float16).astype(np.float32), blocks["qs"].astype(np.int64)


def brute_isums(dtype: int, w: np.ndarray, a: np.ndarray):
    """isum/msum [m, n, kb] by direct element sums.  w [n, kb], a [m, kb]."""
    if dtype == O.Q4K:
        _, _, sc, mn, q = q4k_fields(w)                        # [n,kb,8], [n,kb,256]
        qa = a["qs"].astype(np.int64)                          # [m,kb,256]
        bs = a["bsums"].astype(np.int64)                       # [m,kb,16]
        prod = np.einsum("nbe,mbe->mnbe", q, qa)               # exact ints
        sub = prod.reshape(prod.shape[:3] + (8, 32)).sum(-1)   # [m,n,kb,8]
        isum = (sub * sc[None]).sum(-1)
        msum = (bs.reshape(bs.shape[:2] + (8, 2)).sum(-1)[:, None] * mn[None]).sum(-1)
        return isum.astype(np.int32), msum.astype(np.int32)
    if dtype == O.Q6K:
        _, sc, q = q6k_fields(w)
        qa = a["qs"].astype(np.int64)
        prod = np.einsum("nbe,mbe->mnbe", q, qa)
        sub = prod.reshape(prod.shape[:3] + (16, 16)).sum(-1)
        isum = (sub * sc[None]).sum(-1)
        return isum.astype(np.int32), np.zeros_like(isum, np.int32)
    if dtype == O.Q8_0:
        _, q = q8_0_fields(w)
        qa = a["qs"].astype(np.int64)
        isum = np.einsum("nbe,mbe->mnb", q, qa)
        return isum.astype(np.int32), np.zeros_like(isum, np.int32)
    raise ValueError(dtype)


def exact_dot64(dtype: int, w: np.ndarray, a: np.ndarray) -> np.ndarray:
    """y[m, n] in float64 from the exact integer sums and the block scales:
    sum_b d_w*d_a*isum - dmin_w*d_a*msum (the value vec_dot rounds)."""
    isum, msum = brute_isums(dtype, w, a)
    if dtype == O.Q8_0:
        dw = w["d"].view(np.float16).astype(np.float64)
        da = a["d"].view(np.float16).astype(np.float64)
        return (dw[None] * da[:, None] * isum).sum(-1)
    dw = w["d"].view(np.float16).astype(np.float64)
    da = a["d"].astype(np.float64)
    y = dw[None] * da[:, None] * isum
    if dtype == O.Q4K:
        dm = w["dmin"].view(np.float16).astype(np.float64)
        y = y - dm[None] * da[:, None] * msum
    return y.sum(-1)


def rel_err(got: np.ndarray, want: np.ndarray) -> float:
    """max |got - want| relative to the reference output's L2 norm."""
    want = np.asarray(want, np.float64)
    return float(np.abs(np.asarray(got, np.float64) - want).max() / max(np.linalg.norm(want), 1e-30))
