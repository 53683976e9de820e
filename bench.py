#!/usr/bin/env python3
"""Throughput of the quantized GEMV path on one MI355X.

A step is one pass of the hot path over one batch: the f32 activation of one
token is quantized on the device (Q8_K / I8_S) and multiplied against one
weight matrix in its native GGUF block layout (matmul_batch,
crates/rusticide-kernels/src/matmul.rs:229-248). Weights rotate over more than
1 GiB of distinct HBM copies, so the 256 MB Infinity Cache cannot serve them:
the figure is HBM bandwidth.

`value` is the whole step (both kernels and the gaps between launches) as
algorithmic GB/s: rows*row_bytes (+32 I2_S trailer) + 4*cols (f32 x) +
4*rows (f32 y). `roofline.achieved` is the same bytes over the GEMV kernel's
own average duration, measured with HIP events on the stream it runs on.

Prints one JSON line on stdout; progress goes to stderr.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "Q4_K/Q6_K/I2_S GEMV GB/s (% HBM peak); decode tok/s on 1 MI355X"
HBM_PEAK_GBS = 8000.0
ROTATE_BYTES = 1.1 * 2 ** 30

WORKLOADS = {
    # name: (type_id, rows, cols, description)
    "q6k_lm_head": (14, 32000, 2048, "Q6_K x f32 GEMV 32000x2048 (TinyLlama lm_head), batch 1"),
    "q6k_ffn_down": (14, 2048, 5632, "Q6_K x f32 GEMV 2048x5632 (TinyLlama ffn_down), batch 1"),
    "q4k_ffn_gate": (12, 5632, 2048, "Q4_K x f32 GEMV 5632x2048 (TinyLlama ffn_gate), batch 1"),
    "i2s_up": (36, 6912, 2560, "I2_S x int8 GEMV 6912x2560 (BitNet 2B4T up/gate), batch 1"),
    "i2s_down": (36, 2560, 6912, "I2_S x int8 GEMV 2560x6912 (BitNet 2B4T down), batch 1"),
    "q4k_32000": (12, 32000, 2048, "Q4_K x f32 GEMV 32000x2048 (lm_head shape in Q4_K), batch 1"),
}
HEADLINE = "q6k_lm_head"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def algorithmic_bytes(type_id: int, rows: int, cols: int) -> int:
    from rusticide_amd import synth
    b = rows * synth.row_bytes(type_id, cols) + 4 * cols + 4 * rows
    return b + (32 if type_id == 36 else 0)


def measure_gpu(ctx, name: str, steps: int, warmup: int):
    import rusticide_amd as R
    from rusticide_amd import hip as H
    from rusticide_amd import synth

    type_id, rows, cols, desc = WORKLOADS[name]
    data = synth.matrix(type_id, rows, cols, seed=1)
    one = R.Matrix.load(ctx, type_id, data, rows, cols)
    ncopies = max(2, math.ceil(ROTATE_BYTES / one.device_bytes))
    mats = [one] + [R.Matrix.load(ctx, type_id, data, rows, cols) for _ in range(ncopies - 1)]
    x = H.DeviceArray.from_numpy(synth.normal_f32(cols, seed=2))
    out = H.DeviceArray(rows)
    stream = ctx.stream
    kind = R.ROW if type_id == 36 else R.SUPER_BLOCK
    B = algorithmic_bytes(type_id, rows, cols)

    def step(i):
        R.matmul_batch_device(ctx, x, 1, [(mats[i % ncopies], out)])

    # whole step: quantize + GEMV, back to back on the context's stream
    for i in range(warmup):
        step(i)
    H.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        step(i)
    H.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1e3 / steps

    # the GEMV kernel alone, per launch, with events on its stream
    q8 = R.Q8(ctx).quantize(x, 1, kind)

    def kernel_avg_us(copies: int) -> float:
        # events bracket `steps` back-to-back launches on the kernel's stream
        start, end = H.Event(), H.Event()
        for i in range(warmup):
            R.dot_matrix_device(mats[i % copies], q8, out)
        start.record(stream)
        for i in range(steps):
            R.dot_matrix_device(mats[i % copies], q8, out)
        end.record(stream)
        H.synchronize()
        return 1e3 * start.elapsed_ms(end) / steps

    cold_us = kernel_avg_us(ncopies)
    warm_us = kernel_avg_us(1)
    gpu_out = out.numpy()
    for m in mats:
        m.free()
    q8.free()
    return {
        "workload": name, "desc": desc, "type_id": type_id, "rows": rows, "cols": cols,
        "bytes": B, "copies": ncopies, "ms_per_step": ms_per_step,
        "step_gbs": B / (ms_per_step * 1e-3) / 1e9,
        "kernel_us": cold_us, "kernel_gbs": B / (cold_us * 1e-6) / 1e9,
        "warm_kernel_us": warm_us, "warm_kernel_gbs": B / (warm_us * 1e-6) / 1e9,
        "data": data, "x": x.numpy(), "gpu_out": gpu_out,
    }


def measure_cpu(res: dict, seconds: float):
    """The oracle (a C restatement of the CPU path) on this host's cores."""
    import oracle as O
    from rusticide_amd import synth

    type_id, rows, cols = res["type_id"], res["rows"], res["cols"]
    threads = max(1, min(16, os.cpu_count() or 1))
    rb = synth.row_bytes(type_id, cols)
    if type_id == 36:
        w = O.Weights.ternary(res["data"][: rows * rb], rb, 0.02)
    else:
        w = O.Weights.blocks(type_id, res["data"], rb)
    out = np.zeros(rows, np.float32)
    O.matvec_batch(res["x"], [(w, out)], threads=threads)  # warm-up
    same = bool(np.array_equal(out.view(np.uint32), res["gpu_out"].view(np.uint32)))
    n, t0 = 0, time.perf_counter()
    while True:
        O.matvec_batch(res["x"], [(w, out)], threads=threads)
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            break
    per = el / n
    cpu = platform.processor() or platform.machine()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {
        "value": round(res["bytes"] / per / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
        "sample": (f"{n} full {rows}x{cols} GEMVs incl. activation quantization, "
                   f"{threads} threads, {el:.2f} s wall on {cpu}; bit-identical to the GPU: {same}"),
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--workloads", default="all", help="comma list, or 'all' / 'headline'")
    ap.add_argument("--cpu-seconds", type=float, default=1.5)
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: the path runs on a single MI355X (asked for "
              f"--gpus {args.gpus}, WORLD_SIZE={world}); multi-GPU sharding is design-only.",
              file=sys.stderr)
        return 2

    import rusticide_amd as R
    default = [n for n in WORKLOADS if n != "q4k_32000"]
    names = default if args.workloads == "all" else (
        [HEADLINE] if args.workloads == "headline" else args.workloads.split(","))
    if HEADLINE not in names:
        names.insert(0, HEADLINE)
    ctx = R.Context(0)
    results = {}
    for name in names:
        log(f"[bench] {name}: {WORKLOADS[name][3]}")
        results[name] = measure_gpu(ctx, name, args.steps, args.warmup)
        r = results[name]
        log(f"[bench]   step {r['ms_per_step'] * 1e3:.2f} us = {r['step_gbs']:.0f} GB/s; kernel "
            f"{r['kernel_us']:.2f} us = {r['kernel_gbs']:.0f} GB/s (HBM, {r['copies']} copies); "
            f"warm {r['warm_kernel_us']:.2f} us = {r['warm_kernel_gbs']:.0f} GB/s")
    h = results[HEADLINE]
    cpu = None if args.no_cpu else measure_cpu(h, args.cpu_seconds)
    if cpu:
        log(f"[bench] cpu baseline: {cpu['value']} GB/s ({cpu['sample']})")
    also = {
        n: {"workload": r["desc"], "step_gbs": round(r["step_gbs"], 1), "kernel_us": round(r["kernel_us"], 3),
            "kernel_gbs": round(r["kernel_gbs"], 1), "hbm_frac": round(r["kernel_gbs"] / HBM_PEAK_GBS, 4),
            "warm_kernel_gbs": round(r["warm_kernel_gbs"], 1), "bytes_per_launch": r["bytes"]}
        for n, r in results.items() if n != HEADLINE
    }
    line = {
        "metric": METRIC,
        "value": round(h["step_gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(h["ms_per_step"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": h["desc"], "rows": h["rows"], "cols": h["cols"], "tokens": 1,
                   "bytes_per_step": h["bytes"], "rotating_copies": h["copies"],
                   "step": "device Q8_K quantize + Q6_K GEMV, weights rotated over >1 GiB"},
        "roofline": {"bound": "hbm", "achieved": round(h["kernel_gbs"], 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(h["kernel_gbs"] / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "gemv_q6k_kernel<1>", "kernel_avg_us": round(h["kernel_us"], 3),
                     "warm_cache_resident_gbs": round(h["warm_kernel_gbs"], 1)},
        "cpu_baseline": cpu,
        "also": also,
    }
    ctx.close()
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
