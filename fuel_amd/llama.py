"""LLaMA-shaped quantized decoder on the gfx950 path (greedy decode, batch 1).

The decode step of fuel's LLaMA layer (fuel-core/src/lazy.rs:7363-7440) with
a KV cache, built from this library's C ABI:

    per layer:  [q|k] = QMatMul_Q4K(rms_norm(x) * attn_gain)        (one launch for both, Wq|Wk stacked)
                v     = QMatMul_Q6K(rms_norm(x) * attn_gain)
                a     = attention(rope(q), cache <- rope(k), v)      (RoPE + f16 cache append fused)
                x    += QMatMul_Q4K(a)                               (split merge + residual fused)
                h     = silu(QMatMul_Q4K(a)) * QMatMul_Q4K(a),  a = rms_norm(x) * ffn_gain
                                                                     (Wg|Wu stacked; one launch, h written)
                x    += QMatMul_down(h)                              (residual fused)
    logits = QMatMul_Q6K(rms_norm(x) * final_gain); next = argmax; x = embed[next]; pos += 1

Five launches per layer (the attention's split kernel; its merge runs inside the
o-projection mat-vec), 162 per token (fuse_oproj=False: the merge as its own
kernel, six per layer, 194 per token; fuse_glu=False: gate|up written and the
SwiGLU product formed in the down projection's activation stage; the same
bits either way).  The position lives in device memory,
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
N_TYPE_SIZE = {N.Q8_0: 34, Q4K: 144, Q6K: 210}
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


# GGUF tensor names of the layer matrices (llama.cpp's LLaMA layout, as the
# lazy loader reads them: fuel-core/src/lazy_quantized_llama.rs:224-236)
GGUF_NAMES = {"wq": "attn_q", "wk": "attn_k", "wv": "attn_v", "wo": "attn_output", "wg": "ffn_gate",
              "wu": "ffn_up", "wd": "ffn_down"}


class LlamaDecoder:
    def __init__(self, dev: RocmDevice, cfg: LlamaConfig, seed: int = 1234, std: float = 0.02, _weights=None,
                 fuse_oproj: bool = True, fuse_glu: bool = True, prefill_fused: bool = True):
        if cfg.head_dim != 128 or cfg.n_heads * cfg.head_dim != cfg.dim:
            raise ValueError("this decoder needs head_dim 128 and n_heads * head_dim == dim")
        self.dev, self.cfg, self.seed, self.std = dev, cfg, seed, std
        self.fuse_oproj, self.fuse_glu = fuse_oproj, fuse_glu
        self.prefill_fused = prefill_fused
        L = lib()
        self.L = L
        d, f, H, HD, Cx = cfg.dim, cfg.ffn, cfg.n_heads, cfg.head_dim, cfg.max_ctx
        if _weights is None:  # random-init weights generated on the device
            self.layers = []
            for li in range(cfg.n_layers):
                dts = cfg.layer_dtypes(li)
                self.layers.append({
                    "wqk": self._quantized(Q4K, [("wq", li), ("wk", li)], d, d), "dt_qk": Q4K,
                    "wv": self._quantized(Q6K, [("wv", li)], d, d), "dt_v": Q6K,
                    "wo": self._quantized(Q4K, [("wo", li)], d, d), "dt_o": Q4K,
                    "wgu": self._quantized(Q4K, [("wg", li), ("wu", li)], f, d), "dt_gu": Q4K,
                    "wd": self._quantized(dts["wd"], [("wd", li)], d, f), "dt_down": dts["wd"],
                })
            self.wout, self.dt_out = self._quantized(Q6K, [("out", None)], cfg.vocab, d), Q6K
            self.embed = fill_normal(dev, (cfg.vocab, d), seed, 1, 0.0, std)
            ones = np.ones(d, np.float32)
            self.attn_gain = [dev.from_numpy(ones) for _ in range(cfg.n_layers)]
            self.ffn_gain = [dev.from_numpy(ones) for _ in range(cfg.n_layers)]
            self.final_gain = dev.from_numpy(ones)
        else:
            (self.layers, self.wout, self.dt_out, self.embed, self.attn_gain, self.ffn_gain,
             self.final_gain) = _weights
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
        self.plen = dev.from_numpy(np.zeros(1, np.int32))  # the prompt length, read by the captured step
        self.work_bytes = int(L.frq_attention_decode_workspace(H, Cx))
        self.work = _Buf(dev, self.work_bytes)
        check(L.frq_memset(dev.handle, C.c_void_p(self.work.ptr), 0, self.work_bytes))
        self.prompt_len = 0
        self.scale = float(np.float32(1.0 / np.sqrt(float(HD))))
        dev.synchronize()

    @classmethod
    def from_gguf(cls, dev: RocmDevice, path: str, max_ctx: int = 768) -> "LlamaDecoder":
        """A decoder over the tensors of a GGUF file in llama.cpp's LLaMA
        layout, uploaded verbatim (quantized blocks in [out, in] order; the
        lazy loader's names and slices, fuel-core/src/lazy_quantized_llama.rs:
        224-260).  Hyper-parameters come from the `{arch}.*` metadata; the
        vocabulary size from token_embd.weight, which is also the output
        matrix when output.weight is absent (tied).  f32 / f16 norm gains are
        widened on the host; a quantized token_embd is dequantized on the
        device (to_float).  Grouped-query attention (head_count_kv !=
        head_count) is not supported by this decoder."""
        from .gguf import GgufFile

        g = GgufFile(path)
        md = g.metadata
        arch = md.get("general.architecture", "llama")

        def meta(key, default=None):
            v = md.get(f"{arch}.{key}", default)
            if v is None:
                raise ValueError(f"gguf: missing metadata {arch}.{key}")
            return v

        heads = int(meta("attention.head_count"))
        if int(md.get(f"{arch}.attention.head_count_kv", heads)) != heads:
            raise ValueError("gguf: grouped-query attention (head_count_kv != head_count) is not supported")
        if "token_embd.weight" not in g.tensors:
            raise ValueError("gguf: missing tensor \"token_embd.weight\"")
        dim = int(meta("embedding_length"))
        cfg = LlamaConfig(dim=dim, n_layers=int(meta("block_count")), n_heads=heads, head_dim=dim // heads,
                          ffn=int(meta("feed_forward_length")), vocab=int(g.tensors["token_embd.weight"].dims[0]),
                          eps=float(meta("attention.layer_norm_rms_epsilon", 1e-5)),
                          rope_theta=float(meta("rope.freq_base", 10000.0)), max_ctx=max_ctx)

        def info(name, rows, cols):
            if name not in g.tensors:
                raise ValueError(f"gguf: missing tensor \"{name}\"")
            t = g.tensors[name]
            if t.dims != (rows, cols):
                raise ValueError(f"gguf: tensor {name} has dims {t.dims}, expected {(rows, cols)}")
            if t.dtype not in (Q4K, Q6K, N.Q8_0):
                raise ValueError(f"gguf: tensor {name} has dtype {t.dtype}; the mat-vec takes Q8_0 / Q4_K / Q6_K")
            return t

        def stacked(names, rows, cols):
            infos = [info(n, rows, cols) for n in names]
            if len({t.dtype for t in infos}) != 1:
                raise ValueError(f"gguf: {names} must share one dtype to be stacked")
            one = infos[0].nbytes
            buf = _Buf(dev, one * len(names))
            for i, n in enumerate(names):
                g.copy_to_device(dev, n, buf.ptr + i * one)
            return buf, infos[0].dtype

        def vec(name, n):
            if name not in g.tensors:
                raise ValueError(f"gguf: missing tensor \"{name}\"")
            t = g.tensors[name]
            raw = g.tensor_bytes(name)
            if t.dtype == N.F32:
                a = raw.view(np.float32)
            elif t.dtype == N.F16:
                a = raw.view(np.float16).astype(np.float32)
            else:
                raise ValueError(f"gguf: norm tensor {name} has dtype {t.dtype} (f32 / f16 expected)")
            if a.size != n:
                raise ValueError(f"gguf: tensor {name} has {a.size} values, expected {n}")
            return dev.from_numpy(a)

        d, f = cfg.dim, cfg.ffn
        layers, ag, fg = [], [], []
        for li in range(cfg.n_layers):
            nm = {k: f"blk.{li}.{v}.weight" for k, v in GGUF_NAMES.items()}
            lw = {}
            lw["wqk"], lw["dt_qk"] = stacked([nm["wq"], nm["wk"]], d, d)
            lw["wv"], lw["dt_v"] = stacked([nm["wv"]], d, d)
            lw["wo"], lw["dt_o"] = stacked([nm["wo"]], d, d)
            lw["wgu"], lw["dt_gu"] = stacked([nm["wg"], nm["wu"]], f, d)
            lw["wd"], lw["dt_down"] = stacked([nm["wd"]], d, f)
            layers.append(lw)
            ag.append(vec(f"blk.{li}.attn_norm.weight", d))
            fg.append(vec(f"blk.{li}.ffn_norm.weight", d))
        out_name = "output.weight" if "output.weight" in g.tensors else "token_embd.weight"
        wout, dt_out = stacked([out_name], cfg.vocab, d)
        et = g.tensors["token_embd.weight"]
        if et.dtype in (N.F32, N.F16):
            embed = vec("token_embd.weight", cfg.vocab * d)
        else:
            qs = g.load_quantized(dev, "token_embd.weight")
            embed = qs.dequantize(cfg.vocab * d)
            del qs
        embed.shape = (cfg.vocab, d)  # rows of the table (the buffer is contiguous)
        dec = cls(dev, cfg, _weights=(layers, wout, dt_out, embed, ag, fg, vec("output_norm.weight", d)))
        g.close()
        return dec

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

        def mat(buf, dt, rows, cols, idx=0):  # (block bytes, (rows, blocks per row), dtype)
            bs = 32 if dt == N.Q8_0 else 256
            n = rows * (cols // bs) * N_TYPE_SIZE[dt]
            return fetch(buf, idx * n, n), (rows, cols // bs), dt

        out = {"embed": self.embed.numpy(), "final_gain": self.final_gain.numpy(), "layers": []}
        out["out"] = mat(self.wout, self.dt_out, cfg.vocab, d)
        for li, lw in enumerate(self.layers):
            out["layers"].append({
                "wq": mat(lw["wqk"], lw["dt_qk"], d, d, 0), "wk": mat(lw["wqk"], lw["dt_qk"], d, d, 1),
                "wv": mat(lw["wv"], lw["dt_v"], d, d), "wo": mat(lw["wo"], lw["dt_o"], d, d),
                "wg": mat(lw["wgu"], lw["dt_gu"], f, d, 0), "wu": mat(lw["wgu"], lw["dt_gu"], f, d, 1),
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
        self.plen.copy_from(np.array([self.prompt_len], np.int32))
        d = cfg.dim
        check(self.L.frq_memcpy_dtod(self.dev.handle, C.c_void_p(self.x.ptr),
                                     C.c_void_p(self.embed.ptr + int(prompt[0]) * d * 4), d * 4))

    STEP_PARTS = ("qkv", "attention", "gate_up", "down", "logits", "argmax")

    def enqueue_step(self, parts=None) -> None:
        """One token: all layers, logits, next token + embedding, pos += 1.
        `parts` (a subset of STEP_PARTS) enqueues only those launches, for
        per-kernel timing; None enqueues the whole step."""
        cfg, L, h = self.cfg, self.L, self.dev.handle
        d, eps = cfg.dim, cfg.eps
        vp = C.c_void_p
        x = vp(self.x.ptr)
        on = (lambda p: True) if parts is None else (lambda p: p in parts)
        for li in range(len(self.layers)):
            self.enqueue_layer(li, parts)
        if on("logits"):
            check(L.frq_qmatmul_fused(h, self.dt_out, 1, cfg.vocab, d, vp(self.wout.ptr), x, d, None,
                                      vp(self.final_gain.ptr), eps, 0, vp(self.logits.ptr), cfg.vocab))
        if on("argmax"):
            check(L.frq_argmax_embed(h, vp(self.logits.ptr), cfg.vocab, vp(self.embed.ptr), d, vp(self.tokens.ptr),
                                     cfg.max_ctx, vp(self.plen.ptr), vp(self.pos.ptr), x))

    def enqueue_layer(self, li: int, parts=None) -> None:
        """Layer li of the step (lazy.rs:7363-7440) on the residual x at
        position pos: its five (or six) launches, `parts` as in enqueue_step."""
        cfg, L, h = self.cfg, self.L, self.dev.handle
        d, f, eps = cfg.dim, cfg.ffn, cfg.eps
        vp = C.c_void_p
        x = vp(self.x.ptr)
        on = (lambda p: True) if parts is None else (lambda p: p in parts)
        lw = self.layers[li]
        ag, fg = vp(self.attn_gain[li].ptr), vp(self.ffn_gain[li].ptr)
        if not on("qkv"):
            pass
        elif self._pair(lw):
            check(L.frq_qmatmul_fused_pair(h, 1, d, x, d, ag, eps, lw["dt_qk"], 2 * d, vp(lw["wqk"].ptr),
                                           vp(self.qk.ptr), lw["dt_v"], d, vp(lw["wv"].ptr), vp(self.v.ptr)))
        else:
            check(L.frq_qmatmul_fused(h, lw["dt_qk"], 1, 2 * d, d, vp(lw["wqk"].ptr), x, d, None, ag, eps, 0,
                                      vp(self.qk.ptr), 2 * d))
            check(L.frq_qmatmul_fused(h, lw["dt_v"], 1, d, d, vp(lw["wv"].ptr), x, d, None, ag, eps, 0,
                                      vp(self.v.ptr), d))
        if not on("attention"):
            pass
        elif self.fuse_oproj:
            check(L.frq_attention_decode_oproj(h, cfg.n_heads, cfg.head_dim, cfg.max_ctx, vp(self.qk.ptr),
                                               vp(self.v.ptr), vp(self.rcos.ptr), vp(self.rsin.ptr),
                                               vp(self.kc[li].ptr), vp(self.vc[li].ptr), vp(self.pos.ptr),
                                               self.scale, vp(self.work.ptr), self.work_bytes, lw["dt_o"],
                                               vp(lw["wo"].ptr), d, x))
        else:
            check(L.frq_attention_decode(h, cfg.n_heads, cfg.head_dim, cfg.max_ctx, vp(self.qk.ptr),
                                         vp(self.v.ptr), vp(self.rcos.ptr), vp(self.rsin.ptr),
                                         vp(self.kc[li].ptr), vp(self.vc[li].ptr), vp(self.pos.ptr), self.scale,
                                         vp(self.work.ptr), self.work_bytes, vp(self.att.ptr)))
            check(L.frq_qmatmul_fused(h, lw["dt_o"], 1, d, d, vp(lw["wo"].ptr), vp(self.att.ptr), d, None, None,
                                      0.0, 1, x, d))
        if self.fuse_glu:
            up = lw["wgu"].ptr + f * (d // (32 if lw["dt_gu"] == N.Q8_0 else 256)) * N_TYPE_SIZE[lw["dt_gu"]]
            if on("gate_up"):
                check(L.frq_qmatmul_fused_glu(h, lw["dt_gu"], 1, f, d, vp(lw["wgu"].ptr), vp(up), x, d, fg, eps,
                                              vp(self.gu.ptr), f))
            if on("down"):
                check(L.frq_qmatmul_fused(h, lw["dt_down"], 1, d, f, vp(lw["wd"].ptr), vp(self.gu.ptr), f, None,
                                          None, 0.0, 1, x, d))
        else:
            if on("gate_up"):
                check(L.frq_qmatmul_fused(h, lw["dt_gu"], 1, 2 * f, d, vp(lw["wgu"].ptr), x, d, None, fg, eps, 0,
                                          vp(self.gu.ptr), 2 * f))
            if on("down"):
                check(L.frq_qmatmul_fused(h, lw["dt_down"], 1, d, f, vp(lw["wd"].ptr), vp(self.gu.ptr), f,
                                          vp(self.gu.ptr + 4 * f), None, 0.0, 1, x, d))

    def prefill(self, prompt) -> None:
        """The prompt as one batch (lazy.rs:7363-7446 at seq = M): every layer
        over all M prompt tokens with the int8-MFMA QMatMul (frq_qmatmul, MFMA
        from M = 16 rows) and the prefill row kernels, instead of M decode
        steps.  Leaves the decoder where M forced steps would: cache rows
        0 .. M-1 filled, the logits of position M-1, tokens[M] their greedy
        pick, x its embedding, pos = M (the next enqueue_step emits token
        M+1).  The values differ from the step-by-step path only by summation
        order (MFMA tiles, one attention pass per query row)."""
        self.start(prompt)
        M = self.prompt_len
        cfg, L, h = self.cfg, self.L, self.dev.handle
        d, f, H, HD, Cx, eps = cfg.dim, cfg.ffn, cfg.n_heads, cfg.head_dim, cfg.max_ctx, cfg.eps
        vp = C.c_void_p
        B = self._batch_buffers(M)
        x, xn, qk, v, att, o, gu, hh = (B[k].ptr for k in ("x", "xn", "qk", "v", "att", "o", "gu", "h"))
        check(L.frq_gather_rows(h, vp(self.embed.ptr), cfg.vocab, d, vp(self.tokens.ptr), M, vp(x)))
        for li, lw in enumerate(self.layers):
            ag, fg = vp(self.attn_gain[li].ptr), vp(self.ffn_gain[li].ptr)
            # (the batched fused QMatMuls take Q4_K / Q6_K weights; others run the separate row kernels)
            fused = self.prefill_fused and M >= 2 and all(lw[t] in (Q4K, Q6K) for t in
                                                          ("dt_qk", "dt_v", "dt_o", "dt_gu", "dt_down"))
            if fused and self._pair(lw):  # RMS norm inside the quantize, once for q|k and v
                check(L.frq_qmatmul_fused_pair(h, M, d, vp(x), d, ag, eps, lw["dt_qk"], 2 * d, vp(lw["wqk"].ptr),
                                               vp(qk), lw["dt_v"], d, vp(lw["wv"].ptr), vp(v)))
            else:
                check(L.frq_rms_norm_rows(h, M, d, vp(x), d, ag, eps, vp(xn), d))
                self._mm(lw["dt_qk"], lw["wqk"], 2 * d, d, xn, qk, M)
                self._mm(lw["dt_v"], lw["wv"], d, d, xn, v, M)
            check(L.frq_rope_append_rows(h, M, H, HD, Cx, vp(qk), 2 * d, vp(v), d, vp(self.rcos.ptr),
                                         vp(self.rsin.ptr), 0, vp(self.kc[li].ptr), vp(self.vc[li].ptr)))
            check(L.frq_attention_prefill(h, M, H, HD, Cx, vp(qk), 2 * d, vp(self.kc[li].ptr), vp(self.vc[li].ptr),
                                          0, self.scale, vp(att), d))
            if fused:  # residual adds in the matmul epilogues, SwiGLU inside the down projection's quantize
                check(L.frq_qmatmul_fused(h, lw["dt_o"], M, d, d, vp(lw["wo"].ptr), vp(att), d, None, None, 0.0, 1,
                                          vp(x), d))
                check(L.frq_qmatmul_fused(h, lw["dt_gu"], M, 2 * f, d, vp(lw["wgu"].ptr), vp(x), d, None, fg, eps, 0,
                                          vp(gu), 2 * f))
                check(L.frq_qmatmul_fused(h, lw["dt_down"], M, d, f, vp(lw["wd"].ptr), vp(gu), 2 * f,
                                          vp(gu + 4 * f), None, 0.0, 1, vp(x), d))
                continue
            self._mm(lw["dt_o"], lw["wo"], d, d, att, o, M)
            check(L.frq_add(h, M * d, vp(o), vp(x)))
            check(L.frq_rms_norm_rows(h, M, d, vp(x), d, fg, eps, vp(xn), d))
            self._mm(lw["dt_gu"], lw["wgu"], 2 * f, d, xn, gu, M)
            check(L.frq_swiglu_rows(h, M, f, vp(gu), 2 * f, vp(hh), f))
            self._mm(lw["dt_down"], lw["wd"], d, f, hh, o, M)
            check(L.frq_add(h, M * d, vp(o), vp(x)))
        # the last prompt row: logits, greedy next token and its embedding, pos = M
        check(L.frq_qmatmul_fused(h, self.dt_out, 1, cfg.vocab, d, vp(self.wout.ptr), vp(x + (M - 1) * d * 4), d,
                                  None, vp(self.final_gain.ptr), eps, 0, vp(self.logits.ptr), cfg.vocab))
        self.pos.copy_from(np.array([M - 1], np.int32))
        check(L.frq_argmax_embed(h, vp(self.logits.ptr), cfg.vocab, vp(self.embed.ptr), d, vp(self.tokens.ptr),
                                 cfg.max_ctx, vp(self.plen.ptr), vp(self.pos.ptr), vp(self.x.ptr)))

    def _mm(self, dt, w, n, k, x_ptr, y_ptr, M) -> None:
        """y [M, n] = x [M, k] . W^T through the QMatMul KernelRef seam."""
        bs = 32 if dt == N.Q8_0 else 256
        check(self.L.frq_qmatmul(self.dev.handle, dt, 1, M, n, k, C.c_void_p(x_ptr), M * k * 4, C.c_void_p(w.ptr),
                                 n * (k // bs) * N_TYPE_SIZE[dt], C.c_void_p(y_ptr), M * n * 4))

    def _batch_buffers(self, M: int) -> dict:
        cap = getattr(self, "_batch_cap", 0)
        if cap < M:
            d, f = self.cfg.dim, self.cfg.ffn
            self._batch = {k: self.dev.alloc((M, n), np.float32) for k, n in
                           (("x", d), ("xn", d), ("qk", 2 * d), ("v", d), ("att", d), ("o", d), ("gu", 2 * f),
                            ("h", f))}
            self._batch_cap = M
        return self._batch

    def _pair(self, lw) -> bool:
        kq = (Q4K, Q6K)
        return lw["dt_qk"] in kq and lw["dt_v"] in kq and self.cfg.dim <= 16384

    def launches_per_step(self) -> int:
        per_layer = 5 if self.fuse_oproj else 6
        return sum(per_layer if self._pair(lw) else per_layer + 1 for lw in self.layers) + 2

    def tokens_host(self) -> np.ndarray:
        return self.tokens.numpy()
