"""Profiling runs behind bench.py's roofline figures (run on the GPU box).

Three rocprofv3 passes over bench.py restricted to one shape:
  1. --kernel-trace --stats      -> average duration of the mat-vec kernel;
  2. --pmc FETCH_SIZE            -> KiB fetched per dispatch;
  3. --pmc WRITE_SIZE            -> KiB written per dispatch;
each pass also runs device copies of a known size, whose counter readings give
the factor that converts FETCH_SIZE / WRITE_SIZE to bytes.  Writes a Markdown
summary and a JSON file (traffic bytes per launch) into --out.

With --leg decode / batched / moe it instead runs one --kernel-trace --stats
pass over that bench.py leg (config 4 decode + batched prompt, config 3
M = 32/128/512 matmuls, config 5 MoE layer) and writes the per-kernel summary.

Usage: python bench_profile.py [--shape 4096x32000] [--leg matvec|decode|batched|moe] [--out DIR]
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import statistics
import subprocess
import sys

ROOT = os.path.dirname(os.path.abspath(__file__))
COPY_BYTES = 256 << 20


def run(cmd: list[str], log: str, limit: int) -> None:
    print("+", " ".join(cmd), flush=True)
    with open(os.path.join(ROOT, log), "w") as f:
        subprocess.run(cmd, check=True, stdout=f, stderr=subprocess.STDOUT, cwd=ROOT, timeout=limit)


def rows(d: str, name: str):
    for f in glob.glob(os.path.join(ROOT, d, "**", name), recursive=True):
        yield from csv.DictReader(open(f))


# one kernel-trace pass per leg: (bench.py arguments, summary file name, title)
LEGS = {
    "decode": (["--decode-only", "--no-cpu"], "decode_7b_q4km",
               "Config 4: 7B Q4_K_M decode (512-token batched prompt, 512 forced steps, 256 greedy tokens)"),
    "batched": (["--shape", "4096x4096", "--steps", "5", "--warmup", "1", "--no-cpu", "--no-decode", "--no-moe"],
                "mmq_batched_m32_m128_m512",
                "Config 3: Q4_K / Q6_K QMatMul at M = 32, 128, 512 (int8 MFMA), 7B layer shapes"),
    "moe": (["--shape", "4096x4096", "--steps", "5", "--warmup", "1", "--no-cpu", "--no-decode", "--no-batched",
             "--no-q6k"], "moe_qwen3_layer", "Config 5: Qwen3-MoE layer (route, gate|up, down, combine) at T = 1/16/512"),
}


# The decode leg under rocprofv3 --kernel-trace ended once with a host SIGSEGV
# about a second after HSA initialisation: a memcpy inside the profiler's HIP
# callback read address 0x4ff7c1700000, reached from a ctypes call made
# directly in decode_leg or LlamaDecoder.prefill (the batched and MoE legs,
# which share the device, stream and graph set-up, trace cleanly).  Its cause
# is not established, so that command is not run again.
REFUSED = {"decode": "the decode leg's kernel trace crashed the profiled process (host SIGSEGV in the "
                     "profiler's HIP callback, cause not established); it is not run again"}


def trace_leg(leg: str, out: str, summarize_only: bool) -> int:
    if leg in REFUSED and not summarize_only:
        raise SystemExit(f"bench_profile: --leg {leg} refused: {REFUSED[leg]}")
    bargs, name, title = LEGS[leg]
    cmd = ["rocprofv3", "--kernel-trace", "--stats", "--output-format", "csv", "-d", f"{out}/{name}", "-o", "run",
           "--", "python3", "bench.py"] + bargs
    if not summarize_only:
        run(cmd, f"{out}/{name}.log", 600)
    stats = list(rows(f"{out}/{name}", "run_kernel_stats.csv"))
    total_ns = sum(float(r["TotalDurationNs"]) for r in stats)
    with open(os.path.join(ROOT, out, f"{name}.md"), "w") as f:
        f.write(f"# {title}\n\n")
        f.write(f"Made by `python3 bench_profile.py --leg {leg}` (repository root, one MI355X), which runs:\n\n")
        f.write(f"`{' '.join(cmd)}`\n\n")
        f.write(f"rocprofv3 --stats kernel summary: {len(stats)} kernels, {total_ns / 1e6:.2f} ms of kernel time "
                "in the whole run (warm-up and checks included).\n\n")
        f.write("| kernel | calls | avg us | min us | max us | total ms | % |\n|---|---|---|---|---|---|---|\n")
        for r in sorted(stats, key=lambda r: -float(r["TotalDurationNs"]))[:24]:
            f.write(f"| `{r['Name'][:110]}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
                    f"{float(r['MinNs']) / 1e3:.2f} | {float(r['MaxNs']) / 1e3:.2f} | "
                    f"{float(r['TotalDurationNs']) / 1e6:.3f} | {float(r['Percentage']):.1f} |\n")
    print(f"wrote {out}/{name}.md", flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--shape", default="4096x32000")
    ap.add_argument("--leg", default="matvec", choices=["matvec"] + sorted(LEGS))
    ap.add_argument("--out", default="gpurun_out/profiles")
    ap.add_argument("--summarize-only", action="store_true", help="re-read existing pass outputs")
    args = ap.parse_args()
    os.makedirs(os.path.join(ROOT, args.out), exist_ok=True)
    out = args.out  # relative to the repository root, where every pass runs
    os.environ.setdefault("TMPDIR", "/tmp")
    if args.leg != "matvec":
        return trace_leg(args.leg, out, args.summarize_only)
    bench = ["python3", "bench.py", "--shape", args.shape, "--steps", "50", "--warmup", "5", "--no-cpu",
             "--no-decode", "--no-batched", "--no-moe", "--no-q6k", "--copy-bytes", str(COPY_BYTES)]
    cmds = {
        "trace": ["rocprofv3", "--kernel-trace", "--stats", "--output-format", "csv", "-d", f"{out}/trace", "-o", "run",
                  "--"] + bench,
        "fetch": ["rocprofv3", "--pmc", "FETCH_SIZE", "--output-format", "csv", "-d", f"{out}/fetch", "-o", "run",
                  "--"] + bench,
        "write": ["rocprofv3", "--pmc", "WRITE_SIZE", "--output-format", "csv", "-d", f"{out}/write", "-o", "run",
                  "--"] + bench,
    }
    if not args.summarize_only:
        for k, c in cmds.items():  # counter passes get a short limit of their own
            run(c, f"{out}/{k}.log", 240 if k == "trace" else 90)

    kname = "qmv_kernel<frq::Q4K"
    durs = [int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
            for r in rows(f"{out}/trace", "run_kernel_trace.csv") if kname in r["Kernel_Name"]]
    stats = [r for r in rows(f"{out}/trace", "run_kernel_stats.csv")]

    def counter(d, cname, pred, first=None):
        sel = sorted(((int(r["Dispatch_Id"]), float(r["Counter_Value"])) for r in rows(d, "run_counter_collection.csv")
                      if r["Counter_Name"].startswith(cname) and pred(r["Kernel_Name"])))
        return [v for _, v in (sel[:first] if first else sel)]

    is_copy = lambda n: "copyBuffer" in n
    is_k = lambda n: kname in n
    # the calibration copies are the first three copy dispatches (bench.py --copy-bytes runs them
    # before it builds the rotated weight copies, which are copies too)
    f_copy = counter(f"{out}/fetch", "FETCH_SIZE", is_copy, first=3)
    w_copy = counter(f"{out}/write", "WRITE_SIZE", is_copy, first=3)
    f_k, w_k = counter(f"{out}/fetch", "FETCH_SIZE", is_k), counter(f"{out}/write", "WRITE_SIZE", is_k)
    # copies of COPY_BYTES: fetch reads COPY_BYTES, write writes COPY_BYTES
    f_scale = COPY_BYTES / statistics.median(f_copy)
    w_scale = COPY_BYTES / statistics.median(w_copy)
    fetch_b = statistics.median(f_k) * f_scale
    write_b = statistics.median(w_k) * w_scale
    k, n = (int(v) for v in args.shape.split("x"))
    algo = n * (k // 256) * 144 + 4 * k + 4 * n
    avg_us = statistics.mean(durs) / 1e3
    res = {
        "shape": args.shape,
        "kernel_avg_us": round(avg_us, 3),
        "kernel_median_us": round(statistics.median(durs) / 1e3, 3),
        "dispatches": len(durs),
        "algorithmic_bytes_per_launch": algo,
        "achieved_GB_s_from_trace": round(algo / avg_us / 1e3, 1),
        "fetch_kib_per_dispatch": statistics.median(f_k),
        "write_kib_per_dispatch": statistics.median(w_k),
        "copy_calibration": {"bytes": COPY_BYTES, "fetch_kib": statistics.median(f_copy),
                             "write_kib": statistics.median(w_copy), "fetch_bytes_per_unit": f_scale,
                             "write_bytes_per_unit": w_scale},
        "traffic_bytes_per_launch": int(fetch_b + write_b),
        "traffic_over_algorithmic": round((fetch_b + write_b) / algo, 4),
        "commands": {k2: " ".join(v) for k2, v in cmds.items()},
    }
    json.dump(res, open(os.path.join(ROOT, out, f"qmv_q4k_{args.shape}_traffic.json"), "w"), indent=1)
    with open(os.path.join(ROOT, out, f"qmv_q4k_{args.shape}.md"), "w") as f:
        f.write(f"# Q4_K mat-vec K x N = {args.shape}, M = 1 (qmv_kernel<Q4K>)\n\n")
        f.write(f"Made by `python3 bench_profile.py --shape {args.shape}` (repository root, one MI355X), "
                "which runs:\n\n")
        for k2, v in cmds.items():
            f.write(f"- {k2}: `{' '.join(v)}`\n")
        f.write(f"\nKernel trace: {len(durs)} dispatches, average {avg_us:.3f} us, median "
                f"{res['kernel_median_us']} us -> {res['achieved_GB_s_from_trace']} GB/s of algorithmic bytes "
                f"({algo} B per launch), {res['achieved_GB_s_from_trace'] / 80:.1f}% of 8 TB/s.\n\n")
        f.write(f"Counters (median per dispatch): FETCH_SIZE {res['fetch_kib_per_dispatch']:.0f}, "
                f"WRITE_SIZE {res['write_kib_per_dispatch']:.1f}.  Copy calibration ({COPY_BYTES} B D2D copy): "
                f"FETCH_SIZE {res['copy_calibration']['fetch_kib']:.0f}, WRITE_SIZE "
                f"{res['copy_calibration']['write_kib']:.0f} -> {f_scale:.1f} and {w_scale:.1f} bytes per unit.\n\n")
        f.write(f"HBM traffic per launch: {res['traffic_bytes_per_launch']} B = "
                f"{res['traffic_over_algorithmic']:.3f} x the algorithmic bytes.\n\n")
        f.write("rocprofv3 --stats kernel summary (top rows):\n\n")
        f.write("| kernel | calls | avg ns | total % |\n|---|---|---|---|\n")
        for r in sorted(stats, key=lambda r: -float(r.get("Percentage", 0) or 0))[:6]:
            f.write(f"| {r['Name'][:90]} | {r['Calls']} | {float(r['AverageNs']):.0f} | {float(r['Percentage']):.1f} |\n")
    print(json.dumps(res), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
