"""Benchmark of the MI355X quantized mat-vec path.

A step is one pass of fuel's QMatMul forward at M = 1 (activation quantize to
Q8K + Q4_K block-dot mat-vec, one fused kernel per matrix) over the four
LLaMA-2-7B layer shapes K x N = 4096x4096, 4096x11008, 11008x4096, 4096x32000.
Inputs are resident in HBM before timing starts; every matrix is rotated over
enough copies (>= 1.2 GB per shape) that each launch streams its weights from
HBM rather than the 256 MB Infinity Cache.  Steps are replayed from HIP graphs
and timed with HIP events on the launch stream.

`value` = algorithmic bytes of one step (Q4_K weight bytes + f32 activations in
+ f32 outputs) / measured time per step.  `roofline` reports the dominant
kernel (the 4096x32000 Q4_K mat-vec) timed alone the same way.  `cpu_baseline`
is the oracle's restatement of fuel's CPU path (matmul<BlockQ4K> with the AVX2
vec_dot) on the host cores, on the same four shapes.

The same shapes are then timed with Q6_K weights (`per_shape_q6k`, the rest
of config 2), and config 3's M = 32/128/512 rows run on both formats
(`batched.Q4_K`, `batched.Q6_K`: the int8-MFMA path).

The same run measures BASELINE config 4 (`decode`): greedy decode of a
random-init LLaMA-2-7B-shaped Q4_K_M-mix decoder after a 512-token prompt,
256 generated tokens timed, with fuel's CPU path (the oracle's restatement)
timed on the same weights and KV state beside it (`decode.cpu_baseline`).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-decode] [--decode-only] [--no-q6k]
"""
from __future__ import annotations

import argparse
import glob
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "Q4_K matvec GB/s (% of HBM peak) + decode tokens/s, 7B-shape, 1 MI355X"
SHAPES = [(4096, 4096), (4096, 11008), (11008, 4096), (4096, 32000)]  # (K, N)
HBM_PEAK_GBS = 8000.0
ROTATE_BYTES = 1.2e9
CPU_COPIES = 4
SEED = 20261201


def say(*a):
    print(*a, file=sys.stderr, flush=True)


def algo_bytes(k: int, n: int, type_size: int = 144, block: int = 256) -> int:
    """Algorithmic bytes of one QMatMul at M = 1: weights + f32 x + f32 y."""
    return n * (k // block) * type_size + 4 * k + 4 * n


def copy_calibration(nbytes: int, reps: int = 3) -> None:
    """Device-to-device copies of a known size: the reference point that
    scales rocprofv3's FETCH_SIZE / WRITE_SIZE counters to bytes."""
    import ctypes as C

    import fuel_amd as F

    dev = F.RocmDevice(0)
    a = dev.alloc((nbytes,), np.uint8)
    b = dev.alloc((nbytes,), np.uint8)
    for _ in range(reps):
        F._native.check(F.lib().frq_memcpy_dtod(dev.handle, C.c_void_p(b.ptr), C.c_void_p(a.ptr), nbytes))
    dev.synchronize()
    dev.close()


TYPE_SIZE = {12: 144, 14: 210}  # GGUF codes: Q4_K, Q6_K
TYPE_NAME = {12: "Q4_K", 14: "Q6_K"}


def make_mats(dev, dtype: int, seed_base: int):
    """The four shapes' weights, N(0,0.02) quantized on the device and copied
    until each shape's rotation exceeds ROTATE_BYTES, plus x [1,K] and y [1,N]."""
    import ctypes as C

    import fuel_amd as F

    lib = F.lib()
    mats = []
    for si, (k, n) in enumerate(SHAPES):
        w32 = F.fill_normal(dev, (n, k), SEED, seed_base + si, 0.0, 0.02)
        q0 = dev.qzeros(n * k, dtype)
        q0.quantize(w32)
        dev.synchronize()
        w32.free()
        nbytes = q0.storage_size_in_bytes()
        copies = max(2, math.ceil(ROTATE_BYTES / nbytes))
        ws = [q0]
        for _ in range(copies - 1):
            q = dev.qzeros(n * k, dtype)
            F._native.check(lib.frq_memcpy_dtod(dev.handle, C.c_void_p(q.device_ptr()), C.c_void_p(q0.device_ptr()), nbytes))
            ws.append(q)
        x = F.fill_normal(dev, (1, k), SEED, seed_base + 100 + si)
        y = dev.alloc((1, n), np.float32)
        mats.append(dict(k=k, n=n, ws=ws, x=x, y=y, nbytes=nbytes, dtype=dtype))
    dev.synchronize()
    return mats


def qmatmul_call(dev, mat, i):
    import ctypes as C

    import fuel_amd as F

    w = mat["ws"][i % len(mat["ws"])]
    F._native.check(F.lib().frq_qmatmul(dev.handle, mat["dtype"], 1, 1, mat["n"], mat["k"],
                                        C.c_void_p(mat["x"].ptr), mat["x"].nbytes, C.c_void_p(w.device_ptr()),
                                        mat["nbytes"], C.c_void_p(mat["y"].ptr), mat["y"].nbytes))


def shape_times(hip, dev, stream, mats):
    """Per-shape mat-vec time: graphs of back-to-back launches over the rotation."""
    e0, e1 = hip.event_create(), hip.event_create()
    per_shape = {}
    for m in mats:
        qmatmul_call(dev, m, 0)
        dev.synchronize()
        Rm = len(m["ws"])
        g = hip.capture(stream, lambda m=m, Rm=Rm: [qmatmul_call(dev, m, r) for r in range(Rm)])
        hip.graph_launch(g, stream)
        reps = max(2, 400 // Rm)
        hip.stream_sync(stream)
        hip.event_record(e0, stream)
        for _ in range(reps):
            hip.graph_launch(g, stream)
        hip.event_record(e1, stream)
        hip.event_sync(e1)
        us = hip.elapsed_ms(e0, e1) * 1e3 / (reps * Rm)
        b = algo_bytes(m["k"], m["n"], TYPE_SIZE[m["dtype"]])
        per_shape[f"{m['k']}x{m['n']}"] = {"us": round(us, 3), "GB_s": round(b / us / 1e3, 1),
                                           "hbm_frac": round(b / us / 1e3 / HBM_PEAK_GBS, 4), "launches": reps * Rm}
        hip.graph_destroy(g)
    return per_shape


def gpu_leg(steps: int, warmup: int, q6k: bool = True):
    import fuel_amd as F
    from fuel_amd.hiprt import HipRuntime

    hip = HipRuntime()
    dev = F.RocmDevice(0)
    stream = hip.stream_create()
    dev.set_stream(stream)

    t0 = time.time()
    mats = make_mats(dev, F.Q4K, 100)
    say(f"[bench] weights generated and quantized on device in {time.time() - t0:.1f}s; "
        f"copies per shape: {[len(m['ws']) for m in mats]}")

    # A step is the four QMatMuls (one per shape, the next weight copy of
    # each).  The warmup steps and the timed steps are each captured into one
    # HIP graph and replayed back to back, the way per-shape times are taken:
    # a graph per step would time the host's graph-launch submissions (about
    # 7 us a step, more than the four kernels' launch gaps) instead of the GPU.
    R = max(len(m["ws"]) for m in mats)
    for m in mats:           # first launches outside capture (workspace sizing, lazy init)
        qmatmul_call(dev, m, 0)
    dev.synchronize()

    def steps_graph(first: int, count: int):
        return hip.capture(stream, lambda: [qmatmul_call(dev, m, (first + i) % R)
                                            for i in range(count) for m in mats])

    e0, e1 = hip.event_create(), hip.event_create()
    g_timed = steps_graph(warmup, steps)
    # the timed graph's one-time set-up (uploaded ahead: its first launch would
    # otherwise carry ~2 us a step of it, measured against a second launch)
    hip.graph_upload(g_timed, stream)
    if warmup > 0:
        g_warm = steps_graph(0, warmup)
        hip.graph_launch(g_warm, stream)
        hip.stream_sync(stream)
        hip.graph_destroy(g_warm)
    hip.stream_sync(stream)
    hip.event_record(e0, stream)
    hip.graph_launch(g_timed, stream)
    hip.event_record(e1, stream)
    hip.event_sync(e1)
    ms_total = hip.elapsed_ms(e0, e1)
    hip.graph_destroy(g_timed)
    ms_per_step = ms_total / steps
    step_bytes = sum(algo_bytes(m["k"], m["n"]) for m in mats)

    per_shape = shape_times(hip, dev, stream, mats)
    batched = {}
    if BATCHED_M:
        batched["Q4_K"] = batched_leg(hip, dev, stream, mats)
    mats.clear()  # frees the rotated weights
    per_shape_q6k = None
    if q6k:  # config 2's Q6_K sweep and config 3's Q6_K rows
        mats = make_mats(dev, F.Q6K, 700)
        per_shape_q6k = shape_times(hip, dev, stream, mats)
        say(f"[bench] Q6_K sweep {per_shape_q6k}")
        if BATCHED_M:
            batched["Q6_K"] = batched_leg(hip, dev, stream, mats)
        mats.clear()
    dev.close()
    return ms_per_step, step_bytes, per_shape, R, batched, per_shape_q6k


BATCHED_M = (2, 4, 8, 16, 32, 128, 512)
INT8_PEAK_TOPS = 5000.0


def batched_leg(hip, dev, stream, mats):
    """QMatMul with M = 32, 128, 512 activation rows at the
    same shapes and rotated weights (the int8-MFMA path), and small batches
    M = 2, 4, 8, 16 (the one-pass small-batch mat-vec below 16 rows).
    Reported as useful TOPS (2 M N K per call) against the dense int8 peak and
    as weight bytes per second."""
    import ctypes as C

    import fuel_amd as F

    lib = F.lib()
    e0, e1 = hip.event_create(), hip.event_create()
    out = {}
    for si, m in enumerate(mats):
        k, n, dt = m["k"], m["n"], m["dtype"]
        for M in BATCHED_M:
            x = F.fill_normal(dev, (M, k), SEED, 300 + 10 * si + BATCHED_M.index(M))
            y = dev.alloc((M, n), np.float32)

            def call(r):
                w = m["ws"][r % len(m["ws"])]
                F._native.check(lib.frq_qmatmul(dev.handle, dt, 1, M, n, k, C.c_void_p(x.ptr), x.nbytes,
                                                C.c_void_p(w.device_ptr()), m["nbytes"], C.c_void_p(y.ptr), y.nbytes))

            call(0)  # sizes the workspace outside the capture
            dev.synchronize()
            Rm = len(m["ws"])
            g = hip.capture(stream, lambda: [call(r) for r in range(Rm)])
            hip.graph_launch(g, stream)
            reps = max(2, 60 // Rm)
            hip.stream_sync(stream)
            hip.event_record(e0, stream)
            for _ in range(reps):
                hip.graph_launch(g, stream)
            hip.event_record(e1, stream)
            hip.event_sync(e1)
            us = hip.elapsed_ms(e0, e1) * 1e3 / (reps * Rm)
            hip.graph_destroy(g)
            tops = 2.0 * M * n * k / us / 1e6
            out[f"{k}x{n}_M{M}"] = {"us": round(us, 2), "TOPS": round(tops, 1),
                                    "int8_peak_frac": round(tops / INT8_PEAK_TOPS, 4),
                                    "weight_GB_s": round(m["nbytes"] / us / 1e3, 1)}
            x.free()
            y.free()
    return out


MOE_T = (1, 16, 512)


def moe_leg():
    """Qwen3-MoE-style expert layer, 128 experts, top-8 of
    N(0,1) router logits, d 2048, expert FFN 768, Q4_K experts from N(0,0.02);
    T = 1, 16, 512 tokens.  Four copies of the 340 MB expert set are rotated
    (1.36 GB, beyond the Infinity Cache) and every call routes fresh logits.
    Algorithmic bytes: the distinct routed experts' weights + x in + out."""
    import ctypes as C

    import fuel_amd as F
    from fuel_amd.hiprt import HipRuntime

    E, TOPK, D, FFN, COPIES = 128, 8, 2048, 768, 4
    hip = HipRuntime()
    dev = F.RocmDevice(0)
    stream = hip.stream_create()
    dev.set_stream(stream)
    lib = F.lib()

    def experts(rows, cols, stream_id):
        w32 = F.fill_normal(dev, (E, rows, cols), SEED, stream_id, 0.0, 0.02)
        q = dev.qzeros(E * rows * cols, F.Q4K)
        q.quantize(w32)
        dev.synchronize()
        w32.free()
        return q

    sets = [(experts(FFN, D, 400 + 3 * c), experts(FFN, D, 401 + 3 * c), experts(D, FFN, 402 + 3 * c))
            for c in range(COPIES)]
    per_expert = sum(q.storage_size_in_bytes() for q in sets[0]) // E
    e0, e1 = hip.event_create(), hip.event_create()
    res = {}
    for T in MOE_T:
        NL = 8
        x = F.fill_normal(dev, (T, D), SEED, 500 + T)
        logits = [F.fill_normal(dev, (T, E), SEED, 600 + 10 * T + i) for i in range(NL)]
        out = dev.alloc((T, D), np.float32)

        def call(i):
            g, u, d_ = sets[i % COPIES]
            F._native.check(lib.frq_moe_ffn(dev.handle, F.Q4K, T, D, FFN, E, TOPK, C.c_void_p(x.ptr),
                                            C.c_void_p(logits[i % NL].ptr), C.c_void_p(g.device_ptr()),
                                            C.c_void_p(u.device_ptr()), C.c_void_p(d_.device_ptr()),
                                            C.c_void_p(out.ptr)))

        call(0)
        dev.synchronize()
        R = 8
        g = hip.capture(stream, lambda: [call(i) for i in range(R)])
        hip.graph_launch(g, stream)
        hip.stream_sync(stream)
        reps = 10
        hip.event_record(e0, stream)
        for _ in range(reps):
            hip.graph_launch(g, stream)
        hip.event_record(e1, stream)
        hip.event_sync(e1)
        us = hip.elapsed_ms(e0, e1) * 1e3 / (reps * R)
        hip.graph_destroy(g)
        distinct = float(np.mean([len(np.unique(F.moe_route(dev, lg, TOPK)[0])) for lg in logits]))
        nbytes = distinct * per_expert + 2 * T * D * 4
        res[f"T{T}"] = {"us_per_layer": round(us, 2), "distinct_experts_mean": distinct,
                        "algorithmic_bytes": int(nbytes), "GB_s": round(nbytes / us / 1e3, 1),
                        "path": "grouped int8-MFMA" if T * TOPK > E else "indexed mat-vec"}
        x.free()
        out.free()
    dev.close()
    return res


def probe_leg(k: int, n: int, dtype: int, m: int, reps_target: int = 200) -> dict:
    """One QMatMul configuration alone (profiling runs): M rows x [N, K] of
    `dtype`, weights rotated over >= 1.2 GB, graph-replayed, HIP-event timed."""
    import ctypes as C

    import fuel_amd as F
    from fuel_amd.hiprt import HipRuntime

    hip = HipRuntime()
    dev = F.RocmDevice(0)
    stream = hip.stream_create()
    dev.set_stream(stream)
    lib = F.lib()
    w32 = F.fill_normal(dev, (n, k), SEED, 900, 0.0, 0.02)
    q0 = dev.qzeros(n * k, dtype)
    q0.quantize(w32)
    dev.synchronize()
    w32.free()
    nbytes = q0.storage_size_in_bytes()
    R = max(2, math.ceil(ROTATE_BYTES / nbytes))
    ws = [q0]
    for _ in range(R - 1):
        q = dev.qzeros(n * k, dtype)
        F._native.check(lib.frq_memcpy_dtod(dev.handle, C.c_void_p(q.device_ptr()), C.c_void_p(q0.device_ptr()),
                                            nbytes))
        ws.append(q)
    x = F.fill_normal(dev, (m, k), SEED, 901)
    y = dev.alloc((m, n), np.float32)

    def call(i):
        F._native.check(lib.frq_qmatmul(dev.handle, dtype, 1, m, n, k, C.c_void_p(x.ptr), x.nbytes,
                                        C.c_void_p(ws[i % R].device_ptr()), nbytes, C.c_void_p(y.ptr), y.nbytes))

    call(0)
    dev.synchronize()
    g = hip.capture(stream, lambda: [call(i) for i in range(R)])
    hip.graph_launch(g, stream)
    hip.stream_sync(stream)
    reps = max(2, reps_target // R)
    e0, e1 = hip.event_create(), hip.event_create()
    hip.event_record(e0, stream)
    for _ in range(reps):
        hip.graph_launch(g, stream)
    hip.event_record(e1, stream)
    hip.event_sync(e1)
    us = hip.elapsed_ms(e0, e1) * 1e3 / (reps * R)
    hip.graph_destroy(g)
    dev.close()
    tops = 2.0 * m * n * k / us / 1e6
    return {"probe": f"{k}x{n} dtype {dtype} M={m}", "us": round(us, 3), "TOPS": round(tops, 1),
            "int8_peak_frac": round(tops / INT8_PEAK_TOPS, 4), "weight_GB_s": round(nbytes / us / 1e3, 1),
            "calls": reps * R}


READ_WGPC = (1, 2, 4, 8, 16)
READ_UNROLL = (1, 2, 4, 8)
READ_NT = (0, 1)  # plain loads, non-temporal (streaming) loads


def read_ceiling_leg(nbytes: int, shapes=None, reps_target: int = 200) -> dict:
    """The HBM read ceiling of one launch of `nbytes`: frq_probe_read (a
    kernel that only streams the bytes in, no arithmetic) over a rotation of
    >= 1.2 GB of copies, graph-replayed and HIP-event timed like the mat-vec,
    for each launch shape (workgroups per CU x loads in flight per thread x
    cache policy) in `shapes` (default: every one of READ_WGPC x READ_UNROLL x
    READ_NT); the best is the ceiling the mat-vec's roofline fraction is read
    against."""
    import ctypes as C

    import fuel_amd as F
    from fuel_amd.hiprt import HipRuntime

    hip = HipRuntime()
    dev = F.RocmDevice(0)
    stream = hip.stream_create()
    dev.set_stream(stream)
    lib = F.lib()
    R = max(2, math.ceil(ROTATE_BYTES / nbytes))
    bufs = [F.fill_random_bits(dev, nbytes // 4, 0, SEED, 0, 300 + r) for r in range(R)]
    sink = dev.alloc((1,), np.int32)
    dev.synchronize()
    shapes = shapes or [(w, u, nt) for w in READ_WGPC for u in READ_UNROLL for nt in READ_NT]
    e0, e1 = hip.event_create(), hip.event_create()
    res = {}
    for wgpc, unroll, nt in shapes:
        def call(i, wgpc=wgpc, unroll=unroll, nt=nt):
            F._native.check(lib.frq_probe_read(dev.handle, C.c_void_p(bufs[i % R].ptr), nbytes, wgpc, unroll, nt,
                                               C.c_void_p(sink.ptr)))

        call(0)
        dev.synchronize()
        g = hip.capture(stream, lambda: [call(i) for i in range(R)])
        hip.graph_launch(g, stream)
        hip.stream_sync(stream)
        reps = max(2, reps_target // R)
        hip.event_record(e0, stream)
        for _ in range(reps):
            hip.graph_launch(g, stream)
        hip.event_record(e1, stream)
        hip.event_sync(e1)
        us = hip.elapsed_ms(e0, e1) * 1e3 / (reps * R)
        hip.graph_destroy(g)
        res[f"wg_per_cu{wgpc}_unroll{unroll}" + ("_nt" if nt else "")] = {"us": round(us, 3),
                                                                         "GB_s": round(nbytes / us / 1e3, 1)}
    dev.close()
    best = min(res, key=lambda c: res[c]["us"])
    return {"bytes": nbytes, "best_shape": best, "us": res[best]["us"], "GB_s": res[best]["GB_s"],
            "hbm_frac": round(res[best]["GB_s"] / HBM_PEAK_GBS, 4), "shapes": res, "launches_per_shape": reps * R}


DECODE_PROMPT = 512
DECODE_NEW = 256


def decode_leg(new_tokens: int = DECODE_NEW, prompt_len: int = DECODE_PROMPT):
    """random-init LLaMA-2-7B-shaped decoder (Q4_K_M-style
    mix), a 512-token uniform random prompt, greedy decode of `new_tokens`.
    Every step is one replay of a captured HIP graph (162 launches); the
    prompt is run through the same step with its tokens forced.  Timed: the
    `new_tokens` steps that each emit a generated token.  Also timed: the
    prompt as one batch (`LlamaDecoder.prefill`, int8-MFMA projections), with
    its last-position logits against the forced steps'."""
    import fuel_amd as F
    from fuel_amd.hiprt import HipRuntime
    from fuel_amd.llama import LlamaConfig, LlamaDecoder

    cfg = LlamaConfig(max_ctx=prompt_len + new_tokens)
    hip = HipRuntime()
    dev = F.RocmDevice(0)
    stream = hip.stream_create()
    dev.set_stream(stream)
    t0 = time.time()
    dec = LlamaDecoder(dev, cfg, seed=SEED)
    t_build = time.time() - t0
    bits = F.fill_random_bits(dev, prompt_len, 0, SEED, 0, 77).numpy()
    prompt = (bits % cfg.vocab).astype(np.int32)   # uniform ids in [0, vocab)
    # the prompt as one batch (int8-MFMA projections), timed; the forced
    # steps below then rebuild the caches and the decode runs from there
    e0, e1 = hip.event_create(), hip.event_create()
    dec.prefill(prompt)                            # (first call sizes the batch buffers and workspace)
    hip.stream_sync(stream)
    pre_ms = []
    for _ in range(5):                             # median of five prompt passes
        hip.event_record(e0, stream)
        dec.prefill(prompt)
        hip.event_record(e1, stream)
        hip.event_sync(e1)
        pre_ms.append(hip.elapsed_ms(e0, e1))
    prefill_batched_ms = float(np.median(pre_ms))
    logits_prefill = dec.logits.numpy()
    dec.start(prompt)
    hip.stream_sync(stream)
    g = hip.capture(stream, dec.enqueue_step)
    dec.start(prompt)
    hip.event_record(e0, stream)
    for _ in range(prompt_len - 1):              # forced steps: cache rows 0 .. prompt_len-2
        hip.graph_launch(g, stream)
    hip.event_record(e1, stream)
    hip.event_sync(e1)
    prefill_ms = hip.elapsed_ms(e0, e1)
    hip.event_record(e0, stream)
    for _ in range(new_tokens):                  # each step emits one generated token
        hip.graph_launch(g, stream)
    hip.event_record(e1, stream)
    hip.event_sync(e1)
    decode_ms = hip.elapsed_ms(e0, e1)
    tokens = dec.tokens_host()
    # logits of the first generated position, recomputed eagerly for the CPU check
    p0 = prompt_len - 1
    dec.pos.copy_from(np.array([p0], np.int32))
    import ctypes as C
    F._native.check(F.lib().frq_memcpy_dtod(dev.handle, C.c_void_p(dec.x.ptr),
                                            C.c_void_p(dec.embed.ptr + int(tokens[p0]) * cfg.dim * 4), cfg.dim * 4))
    hip.graph_launch(g, stream)
    hip.stream_sync(stream)
    logits0 = dec.logits.numpy()
    hip.graph_destroy(g)
    wbytes = cfg.weight_bytes_per_token()
    mean_ctx = prompt_len + (new_tokens + 1) / 2.0
    kv_bytes = 2 * cfg.n_layers * cfg.dim * 2 * mean_ctx       # f16 K and V rows read per token
    ms_tok = decode_ms / new_tokens
    res = {
        "tokens_per_s": round(new_tokens / (decode_ms * 1e-3), 1),
        "ms_per_token": round(ms_tok, 4),
        "prefill_ms_by_decode_steps": round(prefill_ms, 2),
        "prefill_ms_batched": round(prefill_batched_ms, 2),
        "prefill_tokens_per_s_batched": round(prompt_len / (prefill_batched_ms * 1e-3), 1),
        # logits of the last prompt position, batched prefill vs the forced steps (max |d| / norm)
        "prefill_logits_rel_err_vs_steps": float(np.abs(logits_prefill - logits0).max() / np.linalg.norm(logits0)),
        "weight_bytes_per_token": wbytes,
        "kv_bytes_per_token_mean": int(kv_bytes),
        "hbm_GB_s": round((wbytes + kv_bytes) / (ms_tok * 1e-3) / 1e9, 1),
        "launches_per_token": dec.launches_per_step(),
        "build_s": round(t_build, 1),
        "generated_head": tokens[prompt_len:prompt_len + 8].tolist(),
    }
    return res, dec, dev, tokens, logits0


def counter_refs() -> dict:
    """The committed counter runs (profiles/*_counters.json, bench_profile.py
    --leg counters: rocprofv3 SQ / MFMA / FETCH_SIZE / WRITE_SIZE passes over
    bench.py --probe, separate processes from this one): per probe, the
    kernel's average time, its HBM fraction and counted-traffic ratio, and for
    the int8-MFMA kernels the MFMA-pipe utilisation from
    SQ_INSTS_VALU_MFMA_MOPS_I8 against the 5 POPS int8 peak."""
    out = {}
    for f in sorted(glob.glob(os.path.join(ROOT, "profiles", "*_counters.json"))):
        d = json.load(open(f))
        keep = ("probe", "kernel_avg_us", "hbm_peak_frac", "traffic_over_algorithmic", "useful_int8_peak_frac",
                "mfma_pipe_int8_peak_frac", "mfma_ops_over_useful", "wave_wait_frac")
        out[os.path.basename(f)[:-len("_counters.json")]] = {k: d[k] for k in keep if k in d}
    return out


def decode_breakdown_leg(new_tokens: int = 128, prompt_len: int = DECODE_PROMPT) -> dict:
    """Per-kernel-class time of the config-4 decode step, from HIP events in
    the process: the decoder is run to position prompt_len + new_tokens (the
    prompt forced, then greedy steps), then each class of the step's launches
    (LlamaDecoder.STEP_PARTS: the q|k + v pair, attention with the
    o-projection, gate|up, down, logits, argmax + embedding) is captured alone
    over all layers and replayed; the whole step is timed the same way."""
    import fuel_amd as F
    from fuel_amd.hiprt import HipRuntime
    from fuel_amd.llama import LlamaConfig, LlamaDecoder

    cfg = LlamaConfig(max_ctx=prompt_len + DECODE_NEW)
    hip = HipRuntime()
    dev = F.RocmDevice(0)
    stream = hip.stream_create()
    dev.set_stream(stream)
    dec = LlamaDecoder(dev, cfg, seed=SEED)
    bits = F.fill_random_bits(dev, prompt_len, 0, SEED, 0, 77).numpy()
    dec.start((bits % cfg.vocab).astype(np.int32))
    g = hip.capture(stream, dec.enqueue_step)
    for _ in range(prompt_len - 1 + new_tokens):
        hip.graph_launch(g, stream)
    hip.stream_sync(stream)
    hip.graph_destroy(g)
    e0, e1 = hip.event_create(), hip.event_create()

    pos0 = dec.pos.numpy().copy()

    def timed(parts, reps=20, inner=1):
        # `inner` copies of the class per graph, so that a one-launch class is
        # not timed by the host's graph submissions; the position is put back
        # after each class (the argmax advances it)
        gg = hip.capture(stream, lambda: [dec.enqueue_step(parts) for _ in range(inner)])
        hip.graph_launch(gg, stream)
        hip.stream_sync(stream)
        hip.event_record(e0, stream)
        for _ in range(reps):
            hip.graph_launch(gg, stream)
        hip.event_record(e1, stream)
        hip.event_sync(e1)
        hip.graph_destroy(gg)
        dec.pos.copy_from(pos0)
        return hip.elapsed_ms(e0, e1) * 1e3 / (reps * inner)

    per_layer = {"qkv": 32, "attention": 32, "gate_up": 32, "down": 32, "logits": 1, "argmax": 1}
    res = {"position": prompt_len - 1 + new_tokens, "max_ctx": cfg.max_ctx, "parts": {}}
    for part in dec.STEP_PARTS:
        us = timed({part}, inner=16 if per_layer[part] == 1 else 1)
        res["parts"][part] = {"us_per_token": round(us, 2), "launches": per_layer[part],
                              "us_per_launch": round(us / per_layer[part], 2)}
    full = timed(None)
    res["step_us"] = round(full, 2)
    res["sum_of_parts_us"] = round(sum(v["us_per_token"] for v in res["parts"].values()), 2)
    res["tokens_per_s"] = round(1e6 / full, 1)
    dev.close()
    return res


def cpu_decode_leg(dec, tokens, logits0, target_s: float, prompt_len: int = DECODE_PROMPT):
    """fuel's CPU quantized path (oracle restatement of the decode step, AVX2
    vec_dot) on the same weights and KV state: decode tokens/s on the host
    cores, and the logits of the first generated position against the GPU's."""
    import oracle as O
    from oracle.llama import LlamaConfig as OConfig, OracleLlama

    threads = int(os.environ.get("RAYON_NUM_THREADS") or os.environ.get("OMP_NUM_THREADS") or 0)
    if threads <= 0:
        threads = len(os.sched_getaffinity(0))
    cfg = dec.cfg
    wh = dec.weights_host()

    def blocks(t):
        raw, shape, dt = t
        return np.frombuffer(raw, dtype=O.BLOCK_DTYPE[dt]).reshape(shape)

    w = {"embed": wh["embed"], "final_gain": wh["final_gain"], "out": blocks(wh["out"]), "layers": []}
    for lw in wh["layers"]:
        w["layers"].append({k: (blocks(v) if isinstance(v, tuple) else v) for k, v in lw.items()})
    del wh
    ocfg = OConfig(dim=cfg.dim, n_layers=cfg.n_layers, n_heads=cfg.n_heads, head_dim=cfg.head_dim, ffn=cfg.ffn,
                   vocab=cfg.vocab, eps=cfg.eps, rope_theta=cfg.rope_theta, max_ctx=cfg.max_ctx)
    m = OracleLlama(ocfg, w, threads=threads)
    p0 = prompt_len - 1
    for li in range(cfg.n_layers):               # the GPU's cache rows 0 .. p0-1
        kc, vc = dec.kv_host(li)
        m.kc[li, :, :p0] = kc[:, :p0]
        m.vc[li, :, :p0] = vc[:, :p0]
    times = []
    t_end = time.time() + target_s
    pos = p0
    logits_cpu0 = None
    while (time.time() < t_end or len(times) < 2) and pos < cfg.max_ctx - 1:
        t = time.perf_counter()
        lg = m.step(int(tokens[pos]), pos)       # teacher-forced on the GPU's tokens
        times.append(time.perf_counter() - t)
        if logits_cpu0 is None:
            logits_cpu0 = lg
        pos += 1
    med = float(np.median(times))
    err = float(np.abs(logits0 - logits_cpu0).max() / np.linalg.norm(logits_cpu0))
    return {
        "value": round(1.0 / med, 3),
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{len(times)} decode steps of the same 7B-shaped model at positions {p0}..{pos - 1} "
                  f"(KV rows 0..{p0 - 1} copied from the GPU run), median {med * 1e3:.1f} ms/token; "
                  f"oracle restatement of the decode step with matmul<T> AVX2 vec_dot, {threads} OpenMP threads",
        "logits_rel_err_vs_gpu_first_step": err,
        "greedy_agrees_first_step": int(np.argmax(logits_cpu0)) == int(tokens[p0 + 1]),
    }


def host_llc_bytes() -> int:
    """Total last-level (L3) cache of the host, from sysfs: the size of each
    distinct L3 instance (shared_cpu_list) summed; 0 when sysfs has none."""
    seen, total = set(), 0
    for idx in glob.glob("/sys/devices/system/cpu/cpu*/cache/index3"):
        try:
            share = open(os.path.join(idx, "shared_cpu_list")).read().strip()
            size = open(os.path.join(idx, "size")).read().strip()
        except OSError:
            continue
        if share in seen:
            continue
        seen.add(share)
        mult = {"K": 1024, "M": 1024 ** 2}.get(size[-1:], 1)
        total += int(size.rstrip("KM")) * mult
    return total


def cpu_leg(target_s: float):
    """fuel's CPU quantized path (oracle restatement, AVX2 vec_dot) on the host
    cores: median time of repeated 4-shape sweeps."""
    import oracle as O

    threads = int(os.environ.get("RAYON_NUM_THREADS") or os.environ.get("OMP_NUM_THREADS") or 0)
    if threads <= 0:
        threads = len(os.sched_getaffinity(0))
    step_bytes = sum(algo_bytes(k, n) for k, n in SHAPES)
    llc = host_llc_bytes()
    # rotated copies, as on the GPU: at least twice the host's last-level cache
    copies = min(16, max(CPU_COPIES, math.ceil(2 * llc / step_bytes)))
    mats = []
    for si, (k, n) in enumerate(SHAPES):
        w = O.quantize(O.Q4K, O.normal((n, k), SEED, 100 + si, std=0.02))
        mats.append((O.normal((1, k), SEED, 200 + si), [w] + [w.copy() for _ in range(copies - 1)]))
    for x, ws in mats:
        O.matmul(O.Q4K, x, ws[0], avx2=True, threads=threads)
    times = []
    t_end = time.time() + target_s
    i = 0
    while time.time() < t_end or len(times) < 3:
        t = time.perf_counter()
        for x, ws in mats:
            O.matmul(O.Q4K, x, ws[i % copies], avx2=True, threads=threads)
        times.append(time.perf_counter() - t)
        i += 1
    med = float(np.median(times))
    return {
        "value": round(step_bytes / med / 1e9, 2),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "host_llc_bytes": llc,
        "sample": f"{len(times)} sweeps of the 4-shape Q4_K M=1 QMatMul ({step_bytes / 1e6:.1f} MB each, "
                  f"weights rotated over {copies} copies = {copies * step_bytes / 1e6:.0f} MB against a "
                  f"host last-level cache of {llc / 1e6:.0f} MB), "
                  f"median {med * 1e3:.2f} ms; oracle matmul<BlockQ4K> with the AVX2 vec_dot, "
                  f"{threads} OpenMP threads; avx2={'yes' if O.have_avx2() else 'no (scalar)'}",
    }


def cpu_config1_leg(target_s: float):
    """BASELINE config 1 on fuel's CPU path itself: matmul<BlockQ8_0> (the
    oracle restatement with the AVX2 vec_dot_q8_0_q8_0, avx.rs:72-88) of
    x [1, 4096] ~ N(0, 1) against W [4096, 4096] ~ N(0, 0.02) quantized by
    BlockQ8_0::from_float, on the host cores; median of repeated calls, the
    weights rotated over enough copies to exceed twice the host's last-level
    cache."""
    import oracle as O

    threads = int(os.environ.get("RAYON_NUM_THREADS") or os.environ.get("OMP_NUM_THREADS") or 0)
    if threads <= 0:
        threads = len(os.sched_getaffinity(0))
    k = n = 4096
    nbytes = algo_bytes(k, n, 34, 32)
    llc = host_llc_bytes()
    copies = min(16, max(CPU_COPIES, math.ceil(2 * llc / nbytes)))
    w = O.quantize(O.Q8_0, O.normal((n, k), SEED, 300, std=0.02))
    ws = [w] + [w.copy() for _ in range(copies - 1)]
    x = O.normal((1, k), SEED, 301)
    O.matmul(O.Q8_0, x, ws[0], avx2=True, threads=threads)
    times = []
    t_end = time.time() + target_s
    i = 0
    while time.time() < t_end or len(times) < 3:
        t = time.perf_counter()
        O.matmul(O.Q8_0, x, ws[i % copies], avx2=True, threads=threads)
        times.append(time.perf_counter() - t)
        i += 1
    med = float(np.median(times))
    return {
        "value": round(nbytes / med / 1e9, 2),
        "unit": "GB/s",
        "us": round(med * 1e6, 2),
        "cores": threads,
        "kind": "port",
        "sample": f"{len(times)} calls of the Q8_0 [1,4096] x [4096,4096] QMatMul ({nbytes / 1e6:.2f} MB each, "
                  f"weights rotated over {copies} copies), median {med * 1e6:.1f} us; oracle matmul<BlockQ8_0> "
                  f"with the AVX2 vec_dot_q8_0_q8_0, {threads} OpenMP threads; "
                  f"avx2={'yes' if O.have_avx2() else 'no (scalar)'}",
    }


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--shape", action="append", default=None,
                    help="restrict the sweep to KxN (profiling runs); repeatable")
    ap.add_argument("--copy-bytes", type=int, default=0,
                    help="first run device copies of this size (counter calibration)")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-batched", action="store_true", help="skip the config-3 M = 32/128/512 leg")
    ap.add_argument("--no-moe", action="store_true", help="skip the config-5 MoE leg")
    ap.add_argument("--no-q6k", action="store_true", help="skip the Q6_K sweep and Q6_K batched rows")
    ap.add_argument("--decode-only", action="store_true", help="run only the config-4 decode legs")
    ap.add_argument("--decode-breakdown", action="store_true",
                    help="time each kernel class of the config-4 decode step (HIP events) and print its JSON line")
    ap.add_argument("--probe", default=None, metavar="K,N,DTYPE,M",
                    help="time one QMatMul configuration alone (profiling runs) and print its JSON line")
    ap.add_argument("--probe-read", default=None, metavar="BYTES[,WG_PER_CU,UNROLL[,NT]]",
                    help="time the streaming-read probe over BYTES (every launch shape, or the one given) "
                         "and print its JSON line")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X: --gpus {args.gpus} is not supported "
              "(this build has no multi-GPU path; the sharding design is documented only)", file=sys.stderr)
        return 2

    if args.decode_breakdown:
        print(json.dumps(decode_breakdown_leg()), flush=True)
        return 0
    if args.probe:
        k, n, dt, m = (int(v) for v in args.probe.split(","))
        print(json.dumps(probe_leg(k, n, dt, m)), flush=True)
        return 0
    if args.probe_read:
        if args.copy_bytes:
            copy_calibration(args.copy_bytes)
        v = [int(t) for t in args.probe_read.split(",")]
        shape = [(v[1], v[2], v[3] if len(v) > 3 else 0)] if len(v) >= 3 else None
        print(json.dumps(read_ceiling_leg(v[0], shape)), flush=True)
        return 0
    global SHAPES
    if args.shape:
        SHAPES = [tuple(int(v) for v in sh.split("x")) for sh in args.shape]
    if args.copy_bytes:
        copy_calibration(args.copy_bytes)
    if args.decode_only:
        dres, dec, dev, tokens, logits0 = decode_leg()
        say(f"[bench] decode {dres}")
        if not args.no_cpu:
            dres["cpu_baseline"] = cpu_decode_leg(dec, tokens, logits0, args.cpu_seconds)
        print(json.dumps({"metric": "decode tokens/s, LLaMA-2-7B-shaped Q4_K_M mix (BASELINE config 4)",
                          "value": dres["tokens_per_s"], "unit": "tokens/s", "decode": dres}), flush=True)
        return 0
    global BATCHED_M
    if args.no_batched:
        BATCHED_M = ()
    ms_per_step, step_bytes, per_shape, rot, batched, per_shape_q6k = gpu_leg(args.steps, args.warmup,
                                                                              not args.no_q6k)
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    dom_key = "4096x32000" if "4096x32000" in per_shape else next(iter(per_shape))
    dom = per_shape[dom_key]
    dk, dn = (int(v) for v in dom_key.split("x"))
    dom_bytes = algo_bytes(dk, dn)
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "qmv_q4k_%s_traffic.json" % dom_key)
    if os.path.exists(tpath):  # HBM bytes per launch from the committed FETCH/WRITE_SIZE runs
        traffic = json.load(open(tpath)).get("traffic_bytes_per_launch")
    out = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic: Philox-4x32-10 N(0,1) activations, N(0,0.02) weights quantized to Q4_K on the device "
                "by the from_float port (bit-exact with the CPU quantizer)",
        "config": {
            "workload": "Q4_K batch-1 QMatMul sweep at LLaMA-2-7B layer shapes (BASELINE config 2)",
            "shapes_KxN": [f"{k}x{n}" for k, n in SHAPES],
            "m": 1,
            "weight_rotation_copies": rot,
            "step_algorithmic_bytes": step_bytes,
        },
        "hbm_frac": round(value / HBM_PEAK_GBS, 4),
        "per_shape": per_shape,
        "per_shape_q6k": per_shape_q6k,
        "counters_from_profiles": counter_refs(),
        "decode_tokens_per_s": None,
        "roofline": {
            "bound": "hbm",
            "kernel": f"qmv_kernel<Q4K> (fused Q8K quantize + mat-vec), K={dk} N={dn}, M=1",
            "achieved": dom["GB_s"],
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(dom["GB_s"] / HBM_PEAK_GBS, 4),
            "bytes_per_launch": dom_bytes,
            "avg_launch_us": dom["us"],
            "traffic": traffic,
        },
    }
    if dom_key == "4096x32000":  # the read ceiling of a launch that size (pure streaming read, best launch shape)
        rc = read_ceiling_leg(dom_bytes - dom_bytes % 16)
        out["roofline"]["read_ceiling"] = {k: rc[k] for k in ("bytes", "best_shape", "us", "GB_s", "hbm_frac")}
        out["roofline"]["frac_of_read_ceiling"] = round(dom["GB_s"] / rc["GB_s"], 4)
        say(f"[bench] read ceiling {rc}")
    if batched:
        out["batched"] = batched
    if not args.shape:  # BASELINE config 1's QMatMul (Q8_0 [1,4096] x [4096,4096]) on the device
        c1 = probe_leg(4096, 4096, 8, 1)
        c1_bytes = algo_bytes(4096, 4096, 34, 32)
        out["config1_q8_0_4096x4096"] = {"us": c1["us"], "GB_s": round(c1_bytes / c1["us"] / 1e3, 1),
                                         "hbm_frac": round(c1_bytes / c1["us"] / 1e3 / HBM_PEAK_GBS, 4)}
        if not args.no_cpu:  # the same QMatMul on fuel's CPU path, on the host cores
            c1cpu = cpu_config1_leg(min(3.0, args.cpu_seconds))
            out["config1_q8_0_4096x4096"]["cpu_baseline"] = c1cpu
            out["config1_q8_0_4096x4096"]["gpu_over_cpu"] = round(c1cpu["us"] / c1["us"], 1)
        say(f"[bench] config 1 {out['config1_q8_0_4096x4096']}")
    if not args.no_moe:
        out["moe"] = moe_leg()
        say(f"[bench] moe {out['moe']}")
    if not args.no_decode:
        dres, dec, dev, tokens, logits0 = decode_leg()
        say(f"[bench] decode {dres}")
        out["decode_tokens_per_s"] = dres["tokens_per_s"]
        out["decode"] = dres
        if not args.no_cpu:
            dres["cpu_baseline"] = cpu_decode_leg(dec, tokens, logits0, args.cpu_seconds)
            out["decode_cpu_tokens_per_s"] = dres["cpu_baseline"]["value"]
        del dec, dev
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_leg(args.cpu_seconds)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
