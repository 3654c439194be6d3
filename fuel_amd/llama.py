"""LLaMA-shaped quantized decoder on the gfx950 path (greedy decode, batch 1).

The decode step of fuel's LLaMA layer (fuel-core/src/lazy.rs:7363-7440) with
a KV cache, built from this library's C ABI:

    per layer:  [q|k] = QMatMul_Q4K(rms_norm(x) * attn_gain)        (one launch for both, Wq|Wk stacked)
                v     = QMatMul_Q6K(rms_norm(x) * attn_gain)
                a     = attention(rope(q), cache <- rope(k), v)      (RoPE + f16 cache append fused)
                x    += QMatMul_Q4K(a)                               (residual fused)
                [g|u] = QMatMul_Q4K(rms_norm(x) * ffn_gain)         (Wg|Wu stacked)
                x    += QMatMul_down(silu(g) * u)                    (SwiGLU + residual fused)
    logits = QMatMul_Q6K(rms_norm(x) * final_gain); next = argmax; x = embed[next]; pos += 1

Six launches per layer (the attention is two), 194 per token.  The position lives in device memory,
so one captured HIP graph replays every step (prompt tokens are forced while
they last).  Weights follow a Q4_K_M-style mix: Q4_K everywhere except attn_v,
ffn_down of the even layers and the output matrix (Q6_K).  All weights are
generated and quantized on the device (Philox N(0, 0.02), the device from_float).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import _native as N
from ._native import check, lib
from .backend import RocmDevice, fill_normal

Q4K, Q6K = N.Q4K, N.Q6K
LAYER_MATS = ("wq", "wk", "wv", "wo", "wg", "wu", "wd")


@dataclass
class LlamaConfig:
    dim: int = 4096
    n_layers: int = 32
    n_heads: int = 32
    head_dim: int = 128
    ffn: int = 11008
    vocab: int = 32000
    eps: float = 1e-5
    rope_theta: float = 10000.0
    max_ctx: int = 768

    def down_dtype(self, layer: int) -> int:
        return Q6K if layer % 2 == 0 else Q4K

    def layer_dtypes(self, layer: int) -> dict:
        return {"wq": Q4K, "wk": Q4K, "wv": Q6K, "wo": Q4K, "wg": Q4K, "wu": Q4K, "wd": self.down_dtype(layer)}

    def shapes(self) -> dict:
        d, f = self.dim, self.ffn
        return {"wq": (d, d), "wk": (d, d), "wv": (d, d), "wo": (d, d), "wg": (f, d), "wu": (f, d), "wd": (d, f)}

    def weight_bytes_per_token(self) -> int:
        """Quantized weight bytes one decode step streams (all layers + output)."""
        tsz = {Q4K: 144, Q6K: 210}
        total = 0
        for li in range(self.n_layers):
            for m, (n, k) in self.shapes().items():
                total += n * (k // 256) * tsz[self.layer_dtypes(li)[m]]
        return total + self.vocab * (self.dim // 256) * tsz[Q6K]


def weight_stream(layer: int, mat: str) -> int:
    """Philox stream id of a layer matrix (embed = 1, output = 2)."""
    return 16 + 8 * layer + LAYER_MATS.index(mat)


def rope_tables(base: float, n_pos: int, head_dim: int):
    """build_rope_tables (fuel-graph/src/lib.rs:10808-10868): f64 angles, f32 tables."""
    half = head_dim // 2
    inv = np.array([base ** (-2.0 * i / head_dim) for i in range(half)], np.float64)
    th = np.arange(n_pos, dtype=np.float64)[:, None] * inv[None, :]
    c, s = np.cos(th).astype(np.float32), np.sin(th).astype(np.float32)
    return np.concatenate([c, c], 1), np.concatenate([s, s], 1)


class _Buf:
    """Raw device allocation (bytes) owned by the decoder."""

    def __init__(self, dev: RocmDevice, nbytes: int):
        p = C.c_void_p()
        check(lib().frq_malloc(dev.handle, nbytes, C.byref(p)))
        self.dev, self.ptr, self.nbytes = dev, p.value or 0, nbytes

    def free(self):
        if self.ptr:
            lib().frq_free(self.dev.handle, C.c_void_p(self.ptr))
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class LlamaDecoder:
    def __init__(self, dev: RocmDevice, cfg: LlamaConfig, seed: int = 1234, std: float = 0.02):
        if cfg.head_dim != 128 or cfg.n_heads * cfg.head_dim != cfg.dim:
            raise ValueError("this decoder needs head_dim 128 and n_heads * head_dim == dim")
        self.dev, self.cfg, self.seed, self.std = dev, cfg, seed, std
        L = lib()
        self.L = L
        d, f, H, HD, Cx = cfg.dim, cfg.ffn, cfg.n_heads, cfg.head_dim, cfg.max_ctx
        tsz = {Q4K: 144, Q6K: 210}
        self.layers = []
        for li in range(cfg.n_layers):
            dts = cfg.layer_dtypes(li)
            lw = {
                "wqk": self._quantized(Q4K, [("wq", li), ("wk", li)], d, d),
                "wv": self._quantized(Q6K, [("wv", li)], d, d),
                "wo": self._quantized(Q4K, [("wo", li)], d, d),
                "wgu": self._quantized(Q4K, [("wg", li), ("wu", li)], f, d),
                "wd": self._quantized(dts["wd"], [("wd", li)], d, f),
                "dt_down": dts["wd"],
            }
            self.layers.append(lw)
        self.wout = self._quantized(Q6K, [("out", None)], cfg.vocab, d)
        self.embed = fill_normal(dev, (cfg.vocab, d), seed, 1, 0.0, std)
        ones = np.ones(d, np.float32)
        self.attn_gain = [dev.from_numpy(ones) for _ in range(cfg.n_layers)]
        self.ffn_gain = [dev.from_numpy(ones) for _ in range(cfg.n_layers)]
        self.final_gain = dev.from_numpy(ones)
        c, s = rope_tables(cfg.rope_theta, Cx, HD)
        self.rcos, self.rsin = dev.from_numpy(c), dev.from_numpy(s)
        cache_bytes = H * Cx * HD * 2
        self.kc = [_Buf(dev, cache_bytes) for _ in range(cfg.n_layers)]
        self.vc = [_Buf(dev, cache_bytes) for _ in range(cfg.n_layers)]
        self.x = dev.alloc((d,), np.float32)
        self.qk = dev.alloc((2 * d,), np.float32)
        self.v = dev.alloc((d,), np.float32)
        self.att = dev.alloc((d,), np.float32)
        self.gu = dev.alloc((2 * f,), np.float32)
        self.logits = dev.alloc((cfg.vocab,), np.float32)
        self.tokens = dev.alloc((Cx,), np.int32)
        self.pos = dev.alloc((1,), np.int32)
        self.work_bytes = int(L.frq_attention_decode_workspace(H, Cx))
        self.work = _Buf(dev, self.work_bytes)
        check(L.frq_memset(dev.handle, C.c_void_p(self.work.ptr), 0, self.work_bytes))
        self.prompt_len = 0
        self.scale = float(np.float32(1.0 / np.sqrt(float(HD))))
        dev.synchronize()

    # ---- weights ----

    def _quantized(self, dt: int, parts, rows: int, cols: int) -> _Buf:
        """Stacked quantized matrices (each rows x cols) generated on the device."""
        dev, L = self.dev, self.lib_()
        tsz = {Q4K: 144, Q6K: 210}[dt]
        one = rows * (cols // 256) * tsz
        buf = _Buf(dev, one * len(parts))
        for i, (mat, li) in enumerate(parts):
            stream = 2 if mat == "out" else weight_stream(li, mat)
            w32 = fill_normal(dev, (rows, cols), self.seed, stream, 0.0, self.std)
            q = dev.qzeros(rows * cols, dt)
            q.quantize(w32)
            w32.free()
            check(L.frq_memcpy_dtod(dev.handle, C.c_void_p(buf.ptr + i * one), C.c_void_p(q.device_ptr()), one))
            dev.synchronize()
            del q
        return buf

    @staticmethod
    def lib_():
        return lib()

    def weights_host(self) -> dict:
        """The block bytes and f32 tables as host arrays (the CPU path's view of
        the same model): {"embed", "out", "final_gain", "layers": [...]}."""
        cfg, L, dev = self.cfg, self.L, self.dev

        def fetch(buf: _Buf, off: int, nbytes: int) -> np.ndarray:
            out = np.empty(nbytes, np.uint8)
            check(L.frq_memcpy_dtoh(dev.handle, out.ctypes.data_as(C.c_void_p), C.c_void_p(buf.ptr + off), nbytes))
            return out

        d, f = cfg.dim, cfg.ffn
        tsz = {Q4K: 144, Q6K: 210}

        def mat(buf, dt, rows, cols, idx=0):  # (block bytes, (rows, blocks per row), dtype)
            n = rows * (cols // 256) * tsz[dt]
            return fetch(buf, idx * n, n), (rows, cols // 256), dt

        out = {"embed": self.embed.numpy(), "final_gain": self.final_gain.numpy(), "layers": []}
        out["out"] = mat(self.wout, Q6K, cfg.vocab, d)
        for li, lw in enumerate(self.layers):
            out["layers"].append({
                "wq": mat(lw["wqk"], Q4K, d, d, 0), "wk": mat(lw["wqk"], Q4K, d, d, 1),
                "wv": mat(lw["wv"], Q6K, d, d), "wo": mat(lw["wo"], Q4K, d, d),
                "wg": mat(lw["wgu"], Q4K, f, d, 0), "wu": mat(lw["wgu"], Q4K, f, d, 1),
                "wd": mat(lw["wd"], lw["dt_down"], d, f),
                "attn_gain": self.attn_gain[li].numpy(), "ffn_gain": self.ffn_gain[li].numpy(),
            })
        return out

    def kv_host(self, layer: int):
        """f16 caches of one layer as float32 [heads, max_ctx, head_dim]."""
        cfg = self.cfg
        shape = (cfg.n_heads, cfg.max_ctx, cfg.head_dim)
        res = []
        for buf in (self.kc[layer], self.vc[layer]):
            h = np.empty(shape, np.float16)
            check(self.L.frq_memcpy_dtoh(self.dev.handle, h.ctypes.data_as(C.c_void_p), C.c_void_p(buf.ptr),
                                         h.nbytes))
            res.append(h.astype(np.float32))
        return res

    # ---- decoding ----

    def start(self, prompt) -> None:
        """Load the prompt, put its first token's embedding in x, pos = 0."""
        cfg = self.cfg
        prompt = np.asarray(prompt, np.int32)
        if prompt.size < 1 or prompt.size > cfg.max_ctx:
            raise ValueError(f"prompt of {prompt.size} tokens (1..{cfg.max_ctx})")
        if prompt.min() < 0 or prompt.max() >= cfg.vocab:
            raise ValueError("prompt token outside the vocabulary")
        toks = np.zeros(cfg.max_ctx, np.int32)
        toks[:prompt.size] = prompt
        self.tokens.copy_from(toks)
        self.pos.copy_from(np.zeros(1, np.int32))
        self.prompt_len = int(prompt.size)
        d = cfg.dim
        check(self.L.frq_memcpy_dtod(self.dev.handle, C.c_void_p(self.x.ptr),
                                     C.c_void_p(self.embed.ptr + int(prompt[0]) * d * 4), d * 4))

    def enqueue_step(self) -> None:
        """One token: all layers, logits, next token + embedding, pos += 1."""
        cfg, L, h = self.cfg, self.L, self.dev.handle
        d, f, eps = cfg.dim, cfg.ffn, cfg.eps
        vp = C.c_void_p
        x = vp(self.x.ptr)
        for li, lw in enumerate(self.layers):
            ag, fg = vp(self.attn_gain[li].ptr), vp(self.ffn_gain[li].ptr)
            check(L.frq_qmatmul_fused_pair(h, 1, d, x, d, ag, eps, Q4K, 2 * d, vp(lw["wqk"].ptr), vp(self.qk.ptr),
                                           Q6K, d, vp(lw["wv"].ptr), vp(self.v.ptr)))
            check(L.frq_attention_decode(h, cfg.n_heads, cfg.head_dim, cfg.max_ctx, vp(self.qk.ptr), vp(self.v.ptr),
                                         vp(self.rcos.ptr), vp(self.rsin.ptr), vp(self.kc[li].ptr),
                                         vp(self.vc[li].ptr), vp(self.pos.ptr), self.scale, vp(self.work.ptr),
                                         self.work_bytes, vp(self.att.ptr)))
            check(L.frq_qmatmul_fused(h, Q4K, 1, d, d, vp(lw["wo"].ptr), vp(self.att.ptr), d, None, None, 0.0, 1, x, d))
            check(L.frq_qmatmul_fused(h, Q4K, 1, 2 * f, d, vp(lw["wgu"].ptr), x, d, None, fg, eps, 0,
                                      vp(self.gu.ptr), 2 * f))
            check(L.frq_qmatmul_fused(h, lw["dt_down"], 1, d, f, vp(lw["wd"].ptr), vp(self.gu.ptr), f,
                                      vp(self.gu.ptr + 4 * f), None, 0.0, 1, x, d))
        check(L.frq_qmatmul_fused(h, Q6K, 1, cfg.vocab, d, vp(self.wout.ptr), x, d, None, vp(self.final_gain.ptr),
                                  eps, 0, vp(self.logits.ptr), cfg.vocab))
        check(L.frq_argmax_embed(h, vp(self.logits.ptr), cfg.vocab, vp(self.embed.ptr), d, vp(self.tokens.ptr),
                                 cfg.max_ctx, self.prompt_len, vp(self.pos.ptr), x))

    def launches_per_step(self) -> int:
        return 6 * self.cfg.n_layers + 2

    def tokens_host(self) -> np.ndarray:
        return self.tokens.numpy()
