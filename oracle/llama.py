"""CPU restatement of fuel's quantized LLaMA decode step -- TEST INFRASTRUCTURE ONLY.

Used by tests/ and by bench.py's cpu_baseline leg (the decode tokens/s of
fuel's CPU path on the host cores); nothing in fuel_amd/ imports it.

One token at position `pos` through `LlamaModel::apply_layer`
(fuel-core/src/lazy.rs:7363-7440) with a KV cache, then the final
RmsNorm (:7360), the output projection and the greedy argmax:

    xn = rms_norm(x) * attn_gain                   byte_kernels.rs:2339-2368, lazy.rs:10330-10346
    q, k, v = QMatMul(xn)                           k_quants.rs:2284-2331 (matmul<T>)
    q, k = rope(q), rope(k)                         byte_kernels.rs:1885-1964, tables fuel-graph lib.rs:10808
    cache[pos] = k, v                               (rounded to f16, the cache dtype of this build)
    a = softmax((q . k_j) * 1/sqrt(hd)) . v_j       lazy.rs:7416-7422, byte_kernels.rs:2259-2305
    x = x + QMatMul_o(a)                            lazy.rs:7426
    xn = rms_norm(x) * ffn_gain
    x = x + QMatMul_down(silu(QMatMul_gate(xn)) * QMatMul_up(xn))   lazy.rs:7431-7439
    logits = QMatMul_out(rms_norm(x) * final_gain); next = argmax(logits)   byte_kernels.rs:8246

Weights are GGUF block arrays ([out, in / block] per matrix); the layer
matmuls run through the oracle's matmul<T> (AVX2 vec_dot), i.e. fuel's CPU
quantized path.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import Q4K, Q6K, argmax, attention_decode, matmul, rms_norm, rope, rope_tables


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
        """Q4_K_M-style mix: Q6_K ffn_down on the even layers, Q4_K on the odd."""
        return Q6K if layer % 2 == 0 else Q4K


LAYER_MATS = ("wq", "wk", "wv", "wo", "wg", "wu", "wd")


def layer_dtypes(cfg: LlamaConfig, layer: int) -> dict:
    return {"wq": Q4K, "wk": Q4K, "wv": Q6K, "wo": Q4K, "wg": Q4K, "wu": Q4K, "wd": cfg.down_dtype(layer)}


class OracleLlama:
    """weights: {"embed": f32 [vocab, dim], "out": Q6K blocks [vocab, dim/256],
    "final_gain": f32 [dim], "layers": [ {wq, wk, wv, wo, wg, wu, wd (blocks),
    attn_gain, ffn_gain (f32)} ]}."""

    def __init__(self, cfg: LlamaConfig, weights: dict, threads: int = 0):
        self.cfg = cfg
        self.w = weights
        self.threads = threads
        L, H, C, D = cfg.n_layers, cfg.n_heads, cfg.max_ctx, cfg.head_dim
        self.kc = np.zeros((L, H, C, D), np.float32)
        self.vc = np.zeros((L, H, C, D), np.float32)
        self.cos, self.sin = rope_tables(cfg.rope_theta, 0, C, D)
        self.scale = np.float32(1.0 / np.sqrt(float(D)))

    def _mm(self, dt, x, w):
        return matmul(dt, x[None], w, avx2=True, threads=self.threads)[0]

    def layer(self, li: int, x: np.ndarray, pos: int) -> np.ndarray:
        """apply_layer li (lazy.rs:7363-7440) on the residual x [dim] of the
        token at `pos`: appends its k, v to cache row pos, returns the new x."""
        cfg = self.cfg
        H, D = cfg.n_heads, cfg.head_dim
        lw = self.w["layers"][li]
        cs, sn = self.cos[pos:pos + 1], self.sin[pos:pos + 1]
        dts = layer_dtypes(cfg, li)
        xn = rms_norm(x, lw["attn_gain"], cfg.eps)
        q = self._mm(dts["wq"], xn, lw["wq"])
        k = self._mm(dts["wk"], xn, lw["wk"])
        v = self._mm(dts["wv"], xn, lw["wv"])
        q = rope(q.reshape(H, 1, D), cs, sn).reshape(H, D)
        k = rope(k.reshape(H, 1, D), cs, sn).reshape(H, D)
        self.kc[li, :, pos] = k.astype(np.float16).astype(np.float32)
        self.vc[li, :, pos] = v.reshape(H, D).astype(np.float16).astype(np.float32)
        a = attention_decode(q, self.kc[li], self.vc[li], pos + 1, float(self.scale)).reshape(-1)
        x = (x + self._mm(dts["wo"], a, lw["wo"])).astype(np.float32)
        xn = rms_norm(x, lw["ffn_gain"], cfg.eps)
        g = self._mm(dts["wg"], xn, lw["wg"])
        u = self._mm(dts["wu"], xn, lw["wu"])
        h = (g / (np.float32(1.0) + np.exp(-g)) * u).astype(np.float32)
        return (x + self._mm(dts["wd"], h, lw["wd"])).astype(np.float32)

    def logits(self, x: np.ndarray) -> np.ndarray:
        """The final RmsNorm (lazy.rs:7360) and the output projection."""
        xn = rms_norm(x, self.w["final_gain"], self.cfg.eps)
        return self._mm(Q6K, xn, self.w["out"])

    def step(self, token: int, pos: int) -> np.ndarray:
        """Logits [vocab] of `token` at position `pos` (the cache holds 0..pos-1)."""
        x = self.w["embed"][token].astype(np.float32).copy()
        for li in range(len(self.w["layers"])):
            x = self.layer(li, x, pos)
        return self.logits(x)

    def prefill(self, tokens, workers: int = 16) -> np.ndarray:
        """The prompt as one batch (apply_layer at seq = M, lazy.rs:7363-7446):
        every layer over all M positions with matmul<T> on M rows, the causal
        attention of each query row over cache rows 0 .. its position (rows in
        parallel threads: the C call releases the GIL), the caches filled as M
        steps would fill them.  Returns the logits of the last position."""
        from concurrent.futures import ThreadPoolExecutor

        cfg = self.cfg
        H, D = cfg.n_heads, cfg.head_dim
        toks = np.asarray(tokens, np.int64)
        M = toks.size
        x = self.w["embed"][toks].astype(np.float32)
        cs, sn = self.cos[:M], self.sin[:M]

        def mm(dt, a, w):
            return matmul(dt, a, w, avx2=True, threads=self.threads)

        with ThreadPoolExecutor(workers) as pool:
            for li, lw in enumerate(self.w["layers"]):
                dts = layer_dtypes(cfg, li)
                xn = rms_norm(x, lw["attn_gain"], cfg.eps)
                q = rope(mm(dts["wq"], xn, lw["wq"]).reshape(M, H, D).transpose(1, 0, 2), cs, sn)  # [H, M, D]
                k = rope(mm(dts["wk"], xn, lw["wk"]).reshape(M, H, D).transpose(1, 0, 2), cs, sn)
                v = mm(dts["wv"], xn, lw["wv"]).reshape(M, H, D).transpose(1, 0, 2)
                self.kc[li, :, :M] = k.astype(np.float16).astype(np.float32)
                self.vc[li, :, :M] = v.astype(np.float16).astype(np.float32)
                kc, vc = self.kc[li], self.vc[li]
                rows = list(pool.map(lambda r: attention_decode(q[:, r], kc, vc, r + 1, float(self.scale)),
                                     range(M)))
                a = np.stack(rows).reshape(M, H * D)
                x = (x + mm(dts["wo"], a, lw["wo"])).astype(np.float32)
                xn = rms_norm(x, lw["ffn_gain"], cfg.eps)
                g = mm(dts["wg"], xn, lw["wg"])
                u = mm(dts["wu"], xn, lw["wu"])
                h = (g / (np.float32(1.0) + np.exp(-g)) * u).astype(np.float32)
                x = (x + mm(dts["wd"], h, lw["wd"])).astype(np.float32)
        xn = rms_norm(x[M - 1], self.w["final_gain"], cfg.eps)
        return self._mm(Q6K, xn, self.w["out"])

    def greedy(self, logits: np.ndarray) -> int:
        return argmax(logits)
