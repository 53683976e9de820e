#!/usr/bin/env python3
"""Throughput of the quantized GEMV path on one MI355X.

A step is one pass of the hot path over one batch: matmul_batch
(crates/rusticide-kernels/src/matmul.rs:229-248) of one f32 token against one
weight matrix in its native GGUF block layout. On the device that is a single
kernel launch: every workgroup quantizes the activation into LDS (Q8_K for
Q4_K/Q6_K, I8_S for I2_S, bit-identical to the CPU path) and then streams its
rows. Weights rotate over more than 1 GiB of distinct HBM copies, so the
256 MB Infinity Cache cannot serve them: the figure is HBM bandwidth.

`value` is algorithmic GB/s of the whole step at wall clock:
rows*row_bytes (+32 I2_S trailer) + 4*cols (f32 x) + 4*rows (f32 y).
`roofline.achieved` is the same bytes over the average duration of the step's
GEMV kernel, measured with HIP events on the stream it is launched on.
`roofline.traffic` is the HBM bytes per launch read from the rocprofv3 counter
summary in profiles/ (FETCH_SIZE + WRITE_SIZE, calibrated on a device copy of
known size), when that summary covers the workload.

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
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "hbm_traffic.json")

WORKLOADS = {
    # name: (type_id, rows, cols, description, kernel the step launches)
    "q6k_lm_head": (14, 32000, 2048, "Q6_K x f32 GEMV 32000x2048 (TinyLlama lm_head), batch 1",
                    "gemv_q6k_kernel<1, 4, 1>"),
    "q6k_ffn_down": (14, 2048, 5632, "Q6_K x f32 GEMV 2048x5632 (TinyLlama ffn_down), batch 1",
                     "gemv_q6k_kernel<1, 4, 4>"),
    "q4k_ffn_gate": (12, 5632, 2048, "Q4_K x f32 GEMV 5632x2048 (TinyLlama ffn_gate), batch 1",
                     "gemv_q4k_kernel<1, 4, 1>"),
    "i2s_up": (36, 6912, 2560, "I2_S x int8 GEMV 6912x2560 (BitNet 2B4T up/gate), batch 1",
               "gemv_i2s_fused_kernel<1, 2>"),
    "i2s_down": (36, 2560, 6912, "I2_S x int8 GEMV 2560x6912 (BitNet 2B4T down), batch 1",
                 "gemv_i2s_fused_kernel<1, 2>"),
    "q4k_32000": (12, 32000, 2048, "Q4_K x f32 GEMV 32000x2048 (lm_head shape in Q4_K), batch 1",
                  "gemv_q4k_kernel<1, 4, 1>"),
}
HEADLINE = "q6k_lm_head"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def algorithmic_bytes(type_id: int, rows: int, cols: int) -> int:
    from rusticide_amd import synth
    b = rows * synth.row_bytes(type_id, cols) + 4 * cols + 4 * rows
    return b + (32 if type_id == 36 else 0)


def load_rotation(ctx, name: str):
    """The workload's matrix, uploaded as many times as it takes to exceed ROTATE_BYTES."""
    import rusticide_amd as R
    from rusticide_amd import synth

    type_id, rows, cols = WORKLOADS[name][:3]
    data = synth.matrix(type_id, rows, cols, seed=1)
    one = R.Matrix.load(ctx, type_id, data, rows, cols)
    ncopies = max(2, math.ceil(ROTATE_BYTES / one.device_bytes))
    return data, [one] + [R.Matrix.load(ctx, type_id, data, rows, cols) for _ in range(ncopies - 1)]


def measure_gpu(ctx, name: str, steps: int, warmup: int):
    import rusticide_amd as R
    from rusticide_amd import hip as H
    from rusticide_amd import synth

    type_id, rows, cols, desc, kernel = WORKLOADS[name]
    data, mats = load_rotation(ctx, name)
    ncopies = len(mats)
    x = H.DeviceArray.from_numpy(synth.normal_f32(cols, seed=2))
    out = H.DeviceArray(rows)
    stream = ctx.stream
    B = algorithmic_bytes(type_id, rows, cols)

    def run(copies: int, n: int, first: int = 0) -> None:
        for i in range(first, first + n):
            R.matmul_batch_device(ctx, x, 1, [(mats[i % copies], out)])

    # the timed region: `steps` steps bracketed by device synchronization,
    # with events on the stream the step's one kernel runs on
    run(ncopies, warmup)
    H.synchronize()
    start, end = H.Event(), H.Event()
    t0 = time.perf_counter()
    start.record(stream)
    run(ncopies, steps, warmup)
    end.record(stream)
    H.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1e3 / steps
    kernel_us = 1e3 * start.elapsed_ms(end) / steps
    gpu_out = out.numpy()

    # the same kernel on one cache-resident copy (Infinity Cache), labelled warm
    run(1, warmup)
    start.record(stream)
    run(1, steps)
    end.record(stream)
    H.synchronize()
    warm_us = 1e3 * start.elapsed_ms(end) / steps

    # the unfused form for comparison: the GEMV alone on a pre-quantized activation
    kind = R.ROW if type_id == 36 else R.SUPER_BLOCK
    q8 = R.Q8(ctx).quantize(x, 1, kind)
    for i in range(warmup):
        R.dot_matrix_device(mats[i % ncopies], q8, out)
    start.record(stream)
    for i in range(steps):
        R.dot_matrix_device(mats[i % ncopies], q8, out)
    end.record(stream)
    H.synchronize()
    prequant_us = 1e3 * start.elapsed_ms(end) / steps
    q8.free()
    for m in mats:
        m.free()
    return {
        "workload": name, "desc": desc, "kernel": kernel, "type_id": type_id, "rows": rows, "cols": cols,
        "bytes": B, "copies": ncopies, "ms_per_step": ms_per_step, "step_gbs": B / (ms_per_step * 1e-3) / 1e9,
        "kernel_us": kernel_us, "kernel_gbs": B / (kernel_us * 1e-6) / 1e9,
        "warm_kernel_us": warm_us, "warm_kernel_gbs": B / (warm_us * 1e-6) / 1e9,
        "prequantized_gemv_us": prequant_us,
        "data": data, "x": synth.normal_f32(cols, seed=2), "gpu_out": gpu_out,
    }


def measure_cpu(res: dict, seconds: float):
    """The oracle (a C restatement of the reference CPU path) on this host's cores."""
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


def traffic_for(name: str):
    """HBM bytes per launch of the workload's kernel from the committed counter summary."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
    except (OSError, ValueError):
        return None
    e = t.get("workloads", {}).get(name)
    return None if e is None else e.get("hbm_bytes_per_launch")


def pmc_probe(steps: int) -> int:
    """A short, fixed sequence for `rocprofv3 --pmc` runs: the headline step on
    rotating copies, then device-to-device copies of a known size (the
    calibration for the counters)."""
    import rusticide_amd as R
    from rusticide_amd import hip as H
    from rusticide_amd import synth

    ctx = R.Context(0)
    for name in (HEADLINE, "q4k_ffn_gate", "i2s_up"):
        type_id, rows, cols = WORKLOADS[name][:3]
        _, mats = load_rotation(ctx, name)
        x = H.DeviceArray.from_numpy(synth.normal_f32(cols, seed=2))
        out = H.DeviceArray(rows)
        for i in range(steps):
            R.matmul_batch_device(ctx, x, 1, [(mats[i % len(mats)], out)])
        H.synchronize()
        for m in mats:
            m.free()
        log(f"[pmc] {name}: {steps} steps")
    n = 256 * 2 ** 20
    a, b = H.DeviceArray(n // 4), H.DeviceArray(n // 4)
    a.fill_bytes(1)
    for _ in range(3):
        H.check(H.hip().hipMemcpy(b.ptr, a.ptr, n, H.D2D), "hipMemcpy D2D")
    H.synchronize()
    log(f"[pmc] copy: 3 x {n} bytes device to device")
    ctx.close()
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--workloads", default="all", help="comma list, or 'all' / 'headline'")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--pmc", action="store_true", help="run the short sequence rocprofv3 --pmc profiles")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: the path runs on a single MI355X (asked for "
              f"--gpus {args.gpus}, WORLD_SIZE={world}); multi-GPU sharding is design-only.",
              file=sys.stderr)
        return 2
    if args.pmc:
        return pmc_probe(20)

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
            f"warm {r['warm_kernel_us']:.2f} us = {r['warm_kernel_gbs']:.0f} GB/s; "
            f"pre-quantized GEMV alone {r['prequantized_gemv_us']:.2f} us")
    h = results[HEADLINE]
    cpu = None if args.no_cpu else measure_cpu(h, args.cpu_seconds)
    if cpu:
        log(f"[bench] cpu baseline: {cpu['value']} GB/s ({cpu['sample']})")
    also = {
        n: {"workload": r["desc"], "step_gbs": round(r["step_gbs"], 1), "kernel_us": round(r["kernel_us"], 3),
            "kernel_gbs": round(r["kernel_gbs"], 1), "hbm_frac": round(r["kernel_gbs"] / HBM_PEAK_GBS, 4),
            "warm_kernel_gbs": round(r["warm_kernel_gbs"], 1), "bytes_per_launch": r["bytes"],
            "kernel": r["kernel"], "hbm_traffic_bytes": traffic_for(n)}
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
                   "step": "one launch: in-workgroup Q8_K quantize + Q6_K GEMV, weights rotated over >1 GiB"},
        "roofline": {"bound": "hbm", "achieved": round(h["kernel_gbs"], 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(h["kernel_gbs"] / HBM_PEAK_GBS, 4),
                     "traffic": traffic_for(HEADLINE),
                     "kernel": h["kernel"], "kernel_avg_us": round(h["kernel_us"], 3),
                     "warm_cache_resident_gbs": round(h["warm_kernel_gbs"], 1),
                     "prequantized_gemv_us": round(h["prequantized_gemv_us"], 3)},
        "cpu_baseline": cpu,
        "also": also,
    }
    ctx.close()
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
