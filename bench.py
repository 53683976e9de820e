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
GEMV kernel, measured with HIP events on the stream it is launched on, around
max(`steps`, 200) launches that the host queues behind a bounded hold kernel
(rh_hold_device) so that they run back to back (at least 200, so that the
first launch after the hold does not weigh on a short run's average). Every warm-up makes whole
passes over the rotation of copies and lasts at least 50 ms, so the timed
launches read copies whose pages are mapped and which the Infinity Cache no
longer holds.
`roofline.traffic` is the HBM bytes per launch read from the rocprofv3 counter
summary in profiles/ (FETCH_SIZE + WRITE_SIZE, calibrated on a device copy of
known size), when that summary covers the workload.

`also.prefill_gemm` is the MFMA path at the prefill shapes: Q4_K 5632x2048,
Q6_K 2048x5632 and I2_S 6912x2560 weights against 128, 512 and 2048 tokens (the whole
matmul_batch step and the GEMM kernel alone on pre-quantized activations), as
int8 MFMA utilisation against the 5.0 POPS dense peak, counting
2*rows*cols*tokens operations.

`also.e2e_decode` is the metric's second half: greedy decode of a random-init
TinyLlama-1.1B-shaped model in the Q4_K_M mix (22 layers, 2048 hidden, 32/4
heads of 64, FFN 5632, vocab 32000; Q6_K lm_head and even-layer ffn_down),
a 64-token prompt then 128 greedy tokens (generate.rs:35-124), f32 KV cache.
tok/s = 128 / decode wall time, where decode time is a 129-token generation
less a 1-token one (both include the same prefill, and each pick is followed
by its forward, as generate.rs:83-111 does); the prefill figure is the
prompt's own forward (Decoder.forward_batch) to its last logits, with the
1-token generation beside it. The CPU oracle decodes a
few of the same tokens on the host cores beside it and must pick the same ones.
The model reaches the device as a GGUF file (rusticide_amd.gguf writes it to
a temporary file): `gguf_load` times mapping and parsing it (rh_gguf_open)
and the upload of its tensors to HBM (rh_gguf_model_load), beside a plain
copy from page-locked host memory, the ceiling of any upload.

`cpu_baseline` is the reference's CPU path on this job's share of the host's
cores, restated in C (oracle/): for Q4_K/Q6_K the avx2 restatement of its x86
adapter (rh_avx2.c, eight-row units, the repack done before timing), with the
portable scalar restatement's figure beside it.

Prints one JSON line on stdout; progress goes to stderr.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import platform
import sys
import tempfile
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
                    "gemv_q6k_kernel<1, 8, 1, false, false, 512u, true>"),
    "q6k_ffn_down": (14, 2048, 5632, "Q6_K x f32 GEMV 2048x5632 (TinyLlama ffn_down), batch 1",
                     "gemv_q6k_kernel_pl<1, 1, 4, false, false, 768u, false>"),
    "q4k_ffn_gate": (12, 5632, 2048, "Q4_K x f32 GEMV 5632x2048 (TinyLlama ffn_gate), batch 1",
                     "gemv_q4k_kernel_pl<1, 2, 1, false, false, 512u, true>"),
    "i2s_up": (36, 6912, 2560, "I2_S x int8 GEMV 6912x2560 (BitNet 2B4T up/gate), batch 1",
               "gemv_i2s_one_kernel<256u, 8, 5, true>"),
    "i2s_down": (36, 2560, 6912, "I2_S x int8 GEMV 2560x6912 (BitNet 2B4T down), batch 1",
                 "gemv_i2s_one_kernel<512u, 32, 4, true>"),
    "q4k_32000": (12, 32000, 2048, "Q4_K x f32 GEMV 32000x2048 (lm_head shape in Q4_K), batch 1",
                  "gemv_q4k_kernel<1, 8, 1, false, false, 512u, true>"),
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
    # copies enough that the bytes one launch reads, over all of them, pass
    # ROTATE_BYTES
    ncopies = max(2, math.ceil(ROTATE_BYTES / algorithmic_bytes(type_id, rows, cols)))
    return data, [one] + [R.Matrix.load(ctx, type_id, data, rows, cols) for _ in range(ncopies - 1)]


WARM_MIN_S = 0.05  # every warm-up runs at least this long, whatever --warmup says
HELD_MIN = 200  # launches a held measurement averages over, whatever --steps says


def hold_us_for(launches: int, per_launch_host_us: float = 20.0) -> int:
    """A hold long enough for the host to queue `launches` calls behind it."""
    return int(min(100000, 1000 + per_launch_host_us * launches))


def held_events(ctx, queue, launches: int, per_launch_host_us: float = 20.0):
    """Per-launch device time of `launches` launches queued by `queue()`
    behind a bounded hold (rh_hold_device), so that they run back to back:
    HIP events on the stream the kernels run on, (start, end) around them.
    Returns (us per launch, whether the host finished queueing inside the
    hold, host microseconds per queued launch)."""
    import rusticide_amd as R
    from rusticide_amd import hip as H

    stream = ctx.stream
    hold = hold_us_for(launches, per_launch_host_us)
    start, end = H.Event(), H.Event()
    H.synchronize()
    t = time.perf_counter()
    R.hold(ctx, hold)
    start.record(stream)
    queue()
    end.record(stream)
    queued_s = time.perf_counter() - t
    H.synchronize()
    return 1e3 * start.elapsed_ms(end) / launches, queued_s < hold * 1e-6, queued_s * 1e6 / launches


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
    # the handle arrays are built here, before any timed region: handles[0]
    # starts the rotation at copy 0, handles[1] continues it where `steps`
    # launches from copy 0 leave it
    handles = [R.matrix_handles(mats, 0), R.matrix_handles(mats, steps % ncopies)]

    def run(h, n: int) -> None:
        # the launches are queued from C (one rh_matmul_batch_device each):
        # a Python call per launch can take as long as the kernel itself
        R.matmul_batch_device_repeat_handles(ctx, x, 1, h, out, n)

    # warm-up: whole passes over every copy (each one's pages mapped and read
    # once), at least `warmup` launches and WARM_MIN_S of them; the rotation
    # is back at copy 0 when it ends
    passes, t = max(1, math.ceil(warmup / ncopies)), time.perf_counter()
    run(handles[0], passes * ncopies)
    H.synchronize()
    el = time.perf_counter() - t
    more = math.ceil(max(0.0, WARM_MIN_S - el) / (el / passes))
    if more:
        run(handles[0], more * ncopies)
        H.synchronize()
    warm_launches = (passes + more) * ncopies

    # the timed region: `steps` steps bracketed by device synchronization,
    # wall clock, with events on the stream the step's kernel runs on
    start, end = H.Event(), H.Event()
    H.synchronize()
    t0 = time.perf_counter()
    start.record(stream)
    run(handles[0], steps)
    end.record(stream)
    H.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1e3 / steps
    unheld_us = 1e3 * start.elapsed_ms(end) / steps
    gpu_out = out.numpy()
    # launches continuing the rotation, queued behind a hold: the kernel's
    # back-to-back time per launch, without the host's latency to the first
    # launch, over at least HELD_MIN of them
    nheld = max(steps, HELD_MIN)
    kernel_us, held, host_us = held_events(ctx, lambda: run(handles[1], nheld), nheld)

    # the same kernel on one cache-resident copy (Infinity Cache), labelled warm
    one = R.matrix_handles(mats[:1])
    run(one, max(warmup, 50))
    warm_us = held_events(ctx, lambda: run(one, nheld), nheld)[0]

    # the unfused form for comparison: the GEMV alone on a pre-quantized activation
    kind = R.ROW if type_id == 36 else R.SUPER_BLOCK
    q8 = R.Q8(ctx).quantize(x, 1, kind)
    for i in range(ncopies):
        R.dot_matrix_device(mats[i], q8, out)

    def prequant():
        for i in range(nheld):
            R.dot_matrix_device(mats[i % ncopies], q8, out)

    prequant_us = held_events(ctx, prequant, nheld, per_launch_host_us=60.0)[0]
    q8.free()
    for m in mats:
        m.free()
    return {
        "workload": name, "desc": desc, "kernel": kernel, "type_id": type_id, "rows": rows, "cols": cols,
        "bytes": B, "copies": ncopies, "ms_per_step": ms_per_step, "step_gbs": B / (ms_per_step * 1e-3) / 1e9,
        "kernel_us": kernel_us, "kernel_gbs": B / (kernel_us * 1e-6) / 1e9, "held": held,
        "host_us_per_launch": host_us, "unheld_kernel_us": unheld_us, "warmup_launches": warm_launches,
        "warm_kernel_us": warm_us, "warm_kernel_gbs": B / (warm_us * 1e-6) / 1e9,
        "prequantized_gemv_us": prequant_us,
        "data": data, "x": synth.normal_f32(cols, seed=2), "gpu_out": gpu_out,
    }


def measure_stream_read(ctx, nbytes: int, copies: int, steps: int, warmup: int) -> float:
    """GB/s of a plain streaming read (rh_stream_read_device) of `nbytes` per
    launch, rotated over the same number of copies as the workload: the
    measured ceiling the GEMV kernel is compared with. Warmed up and timed as
    the GEMV is (a whole pass over the copies and WARM_MIN_S, then launches
    queued behind a hold)."""
    import ctypes
    import rusticide_amd as R
    from rusticide_amd import hip as H

    L = R.lib()
    L.rh_stream_read_device.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_size_t,
                                        ctypes.c_size_t, ctypes.c_void_p]
    n = (nbytes + 15) // 16 * 16
    bufs = [H.DeviceArray(n // 4) for _ in range(copies)]
    for b in bufs:
        b.fill_bytes(0x3C)
    ptrs = (ctypes.c_void_p * copies)(*[b.ptr.value for b in bufs])
    sink = H.DeviceArray(2048, dtype=np.uint32)

    # the launches are queued from C: a Python call per launch would take
    # longer than the ~9 us read and leave the GPU idle between launches
    def run(count: int) -> None:
        ctx.check(L.rh_stream_read_device(ctx.handle, ptrs, copies, n, count, sink.ptr))

    passes, t = max(1, math.ceil(warmup / copies)), time.perf_counter()
    run(passes * copies)
    H.synchronize()
    el = time.perf_counter() - t
    more = math.ceil(max(0.0, WARM_MIN_S - el) / (el / passes))
    if more:
        run(more * copies)
    nheld = max(steps, HELD_MIN)
    us = held_events(ctx, lambda: run(nheld), nheld)[0]
    for b in bufs:
        b.free()
    sink.free()
    return n / (us * 1e-6) / 1e9


# The reference's own published single-thread kernel rates for these formats
# (weights per second, 1 token, from its bench baselines cited in `source`),
# with the GB/s they imply at the format's bytes per weight.
REFERENCE_CPU_PUBLISHED = {
    14: {"format": "Q6_K", "bytes_per_weight": 210 / 256,
         "avx2_xeon_w2150b_gw_s": 16.39, "neon_m1_pro_gw_s": 28.82,
         "source": "crates/rusticide-bench/baselines/intel-r-xeon-r-w-2150b-cpu-3-00ghz-20.json:61-64, "
                   "apple-m1-pro-8.json:61-64"},
    12: {"format": "Q4_K", "bytes_per_weight": 144 / 256,
         "avx2_xeon_w2150b_gw_s": 37.92, "neon_m1_pro_gw_s": 47.32,
         "source": "intel-r-xeon-r-w-2150b-cpu-3-00ghz-20.json:45-48, apple-m1-pro-8.json:45-48"},
    36: {"format": "I2_S", "bytes_per_weight": 32 / 128,
         "avx2_xeon_w2150b_gw_s": 7.99, "neon_m1_pro_gw_s": 3.73,
         "source": "intel-r-xeon-r-w-2150b-cpu-3-00ghz-20.json:29-32, apple-m1-pro-8.json:29-32"},
}


def timed_loop(fn, seconds: float):
    """(calls, wall seconds) of calling fn until `seconds` have passed."""
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            return n, el


def measure_cpu(res: dict, seconds: float):
    """The reference's CPU path restated in C on this job's share of the host's
    cores: for Q4_K/Q6_K the avx2 restatement of its x86 adapter (eight-row
    units, vpmaddubsw/vpmaddwd), the baseline `value`; beside it the portable
    scalar restatement, the checker the parity tests use. I2_S has only the
    portable restatement here, which is then the value."""
    import oracle as O
    from rusticide_amd import synth

    type_id, rows, cols = res["type_id"], res["rows"], res["cols"]
    threads = max(1, min(16, os.cpu_count() or 1))
    rb = synth.row_bytes(type_id, cols)
    if type_id == 36:
        w = O.Weights.ternary(res["data"][: rows * rb], rb, 0.02)
    else:
        w = O.Weights.blocks(type_id, res["data"], rb)
    gpu = res["gpu_out"]
    out = np.zeros(rows, np.float32)

    def portable():
        O.matvec_batch(res["x"], [(w, out)], threads=threads)

    avx2 = None
    if type_id in (12, 14) and rows % 8 == 0 and O.Avx2Matrix.available():
        avx2 = O.Avx2Matrix(type_id, res["data"][: rows * rb], rows, rb)
    share = seconds / 2 if avx2 is not None else seconds
    portable()  # warm-up
    same_port = bool(np.array_equal(out.view(np.uint32), gpu.view(np.uint32)))
    n_port, el_port = timed_loop(portable, share)
    port_gbs = res["bytes"] / (el_port / n_port) / 1e9
    cpu = platform.processor() or platform.machine()
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    pub = REFERENCE_CPU_PUBLISHED[type_id]
    published = {
        "reference_adapter": "avx2 (Xeon W-2150B) and neon (Apple M1 Pro), one thread each, published",
        "avx2_gbs_per_thread": round(pub["avx2_xeon_w2150b_gw_s"] * pub["bytes_per_weight"], 2),
        "neon_gbs_per_thread": round(pub["neon_m1_pro_gw_s"] * pub["bytes_per_weight"], 2),
        "source": pub["source"],
    }
    where = (f"{threads} threads, this job's CPU share of the GPU box ({os.cpu_count()} visible), on {cpu}")
    portable_line = {
        "value": round(port_gbs, 3), "unit": "GB/s", "per_thread_gbs": round(port_gbs / threads, 3),
        "sample": f"{n_port} full {rows}x{cols} GEMVs incl. activation quantization, {el_port:.2f} s wall",
        "bit_identical_to_gpu": same_port,
    }
    if avx2 is None:
        return {
            "value": round(port_gbs, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "sample": (f"the portable scalar C restatement of the reference CPU path (the reference has no "
                       f"avx2 kernel restated here for this format): {portable_line['sample']} on {where}; "
                       f"bit-identical to the GPU: {same_port}"),
            "per_thread_gbs": portable_line["per_thread_gbs"],
            "reference_published_per_thread": published,
        }
    out2 = np.zeros(rows, np.float32)

    def vector():
        if not avx2.matvec(res["x"], out2, threads):
            raise RuntimeError("the avx2 restatement refused the activation")

    vector()  # warm-up
    same_avx2 = bool(np.array_equal(out2.view(np.uint32), gpu.view(np.uint32)))
    n_v, el_v = timed_loop(vector, share)
    avx2.close()
    v_gbs = res["bytes"] / (el_v / n_v) / 1e9
    return {
        "value": round(v_gbs, 3), "unit": "GB/s", "cores": threads, "kind": "port",
        "label": "avx2 restatement",
        "sample": (f"the avx2 C restatement of the reference's x86 adapter (eight-row units, "
                   f"vpmaddubsw/vpmaddwd, its repack done before timing): {n_v} full {rows}x{cols} GEMVs "
                   f"incl. activation quantization, {el_v:.2f} s wall on {where}; "
                   f"bit-identical to the GPU: {same_avx2}"),
        "per_thread_gbs": round(v_gbs / threads, 3),
        "portable_restatement": portable_line,
        "reference_published_per_thread": published,
    }


INT8_PEAK_TOPS = 5000.0


GEMM_WORKLOADS = (
    (12, 5632, 2048, "Q4_K 5632x2048 (TinyLlama ffn_gate)"),
    (14, 2048, 5632, "Q6_K 2048x5632 (TinyLlama ffn_down)"),
    (36, 6912, 2560, "I2_S 6912x2560 (BitNet 2B4T up/gate)"),
)


def measure_gemm(ctx, token_counts=(128, 512, 2048), reps: int = 20):
    """Prefill GEMMs (int8 MFMA): the k-quant path on the ffn_gate shape in
    Q4_K and the ffn_down shape in Q6_K, and the ternary path on the BitNet
    up/gate shape."""
    import rusticide_amd as R
    from rusticide_amd import hip as H
    from rusticide_amd import synth

    res = []
    for type_id, rows, cols, desc in GEMM_WORKLOADS:
        data = synth.i2s_matrix(rows, cols, seed=1) if type_id == 36 else synth.matrix(type_id, rows, cols, seed=1)
        mats = [R.Matrix.load(ctx, type_id, data, rows, cols) for _ in range(4)]
        kind = R.ROW if type_id == 36 else R.SUPER_BLOCK
        for T in token_counts:
            x = H.DeviceArray.from_numpy(synth.normal_f32(T * cols, seed=2))
            out = H.DeviceArray(rows * T)
            q8 = R.Q8(ctx).quantize(x, T, kind)

            def timed(fn):
                for i in range(4):
                    fn(i)

                def queue():
                    for i in range(reps):
                        fn(i)

                return held_events(ctx, queue, reps, per_launch_host_us=100.0)[0]

            k_us = timed(lambda i: R.dot_matrix_device(mats[i % 4], q8, out))
            s_us = timed(lambda i: R.matmul_batch_device(ctx, x, T, [(mats[i % 4], out)]))
            ops = 2.0 * rows * cols * T
            res.append({"workload": desc, "tokens": T, "gemm_kernel_us": round(k_us, 2), "step_us": round(s_us, 2),
                        "kernel_tops": round(ops / k_us / 1e6, 1),
                        "mfma_frac": round(ops / k_us / 1e6 / INT8_PEAK_TOPS, 4),
                        "step_tokens_per_s": round(T / s_us * 1e6)})
            q8.free()
        for m in mats:
            m.free()
    return res


def decode_bytes_per_token(model: dict, position: int) -> int:
    """Compulsory HBM bytes of one decode step: every layer matrix, the output
    matrix, the norms, one embedding row and the f32 KV rows read at
    `position` cached positions."""
    from rusticide_amd import synth
    c = model["config"]

    def mbytes(m):
        t, _, rows, cols = m
        return rows * synth.row_bytes(t, cols)

    total = 0
    for b in model["blocks"]:
        total += sum(mbytes(b[k]) for k in ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up",
                                            "ffn_down"))
        total += 4 * 2 * c["embedding_length"]
    out = model["output"] if model.get("output") is not None else model["token_embd"]
    total += mbytes(out) + 4 * c["embedding_length"]
    t, _, _, cols = model["token_embd"]
    total += synth.row_bytes(t, cols)
    kv = c["head_count_kv"] * c["head_dim"]
    total += c["block_count"] * position * kv * 4 * 2
    return total


def measure_h2d(nbytes: int, reps: int = 5) -> float:
    """GB/s of a plain host-to-device copy from page-locked memory: the
    ceiling of any upload from host memory."""
    from rusticide_amd import hip as H

    host, dev = H.PinnedHost(nbytes), H.DeviceArray(nbytes, np.uint8)
    ctypes.memset(host.ptr, 1, nbytes)
    times = []
    for _ in range(reps + 1):
        t = time.perf_counter()
        H.check(H.hip().hipMemcpy(dev.ptr, host.ptr, nbytes, H.H2D), "hipMemcpy H2D")
        times.append(time.perf_counter() - t)
    host.free()
    dev.free()
    return nbytes / float(np.median(times[1:])) / 1e9


def measure_decode(ctx, reps: int, prompt_len: int = 64, new_tokens: int = 128):
    """Greedy decode of the TinyLlama-shaped model on the device."""
    import rusticide_amd as R
    from rusticide_amd import synth

    from rusticide_amd import gguf as G

    t0 = time.perf_counter()
    model = synth.decoder_model(synth.TINYLLAMA, seed=7)
    fd, path = tempfile.mkstemp(suffix=".gguf")
    with os.fdopen(fd, "wb") as fh:
        fh.write(G.decoder_gguf(model))
    size = os.path.getsize(path)
    log(f"[bench] e2e: model and its {size / 1e6:.0f} MB GGUF file written in {time.perf_counter() - t0:.1f} s")
    # the file's way onto the device: map and parse it (rh_gguf_open), then
    # every tensor checked and uploaded (rh_gguf_model_load); the file is in
    # the page cache after the first round
    parse_s, upload_s = [], []
    for _ in range(4):
        t = time.perf_counter()
        f = G.GgufFile.load(path)
        parse_s.append(time.perf_counter() - t)
        t = time.perf_counter()
        gm = G.GgufModel(ctx, f)
        upload_s.append(time.perf_counter() - t)
        gm.free()
        f.close()
    f = G.GgufFile.load(path)
    gm = G.GgufModel(ctx, f)
    dec = gm.decoder()
    h2d = measure_h2d(256 << 20)
    load = {"file_bytes": size, "tensors": f.tensor_count, "open_parse_ms": float(np.median(parse_s[1:])) * 1e3,
            "upload_ms": float(np.median(upload_s[1:])) * 1e3, "first_upload_ms": upload_s[0] * 1e3,
            "pinned_h2d_gbs": h2d}
    load["upload_gbs"] = size / (load["upload_ms"] * 1e-3) / 1e9
    load["frac_of_pinned_h2d"] = load["upload_gbs"] / h2d
    log(f"[bench] e2e: GGUF open+parse {load['open_parse_ms']:.2f} ms, upload {load['upload_ms']:.1f} ms "
        f"({load['upload_gbs']:.1f} GB/s host to HBM; a pinned-buffer copy reaches {h2d:.1f} GB/s)")
    prompt = np.random.default_rng(1).integers(0, synth.TINYLLAMA["vocab_size"], prompt_len).astype(np.uint32)
    tokens = dec.generate_greedy(prompt, new_tokens + 1)  # warm-up
    decode_s, gen1_s, prefill_s = [], [], []
    for _ in range(reps):
        t = time.perf_counter()
        dec.generate_greedy(prompt, 1)
        t1 = time.perf_counter() - t
        t = time.perf_counter()
        got = dec.generate_greedy(prompt, new_tokens + 1)
        tn = time.perf_counter() - t
        assert np.array_equal(got, tokens), "greedy decode is not deterministic"
        decode_s.append(tn - t1)
        gen1_s.append(t1)
        # the prefill alone: the prompt's forward to its last logits (a
        # one-token generation also picks and, as generate.rs:83-111 does
        # after every pick, runs the picked token's forward)
        dec.reset()
        t = time.perf_counter()
        dec.forward_batch(prompt, 0)
        prefill_s.append(time.perf_counter() - t)
    dec.close()
    gm.free()
    f.close()
    os.unlink(path)
    d = float(np.median(decode_s))
    per_token = decode_bytes_per_token(model, prompt_len + new_tokens // 2)
    return {
        "model": model, "prompt": prompt, "tokens": tokens[:new_tokens],
        "tok_s": new_tokens / d, "us_per_token": d / new_tokens * 1e6,
        "prefill_ms": float(np.median(prefill_s)) * 1e3, "generate_1_ms": float(np.median(gen1_s)) * 1e3,
        "bytes_per_token": per_token,
        "gbs": per_token / (d / new_tokens) / 1e9, "gguf_load": load,
    }


def measure_cpu_decode(res: dict, tokens: int = 8):
    """The oracle's decoder on the host cores: the same prompt's prefill, then
    `tokens` greedy steps, which must pick the device's tokens."""
    import oracle as O

    threads = max(1, min(16, os.cpu_count() or 1))
    cpu = O.Decoder(res["model"], threads=threads)
    t = time.perf_counter()
    got = cpu.generate_greedy(res["prompt"], 1)
    t1 = time.perf_counter() - t
    t = time.perf_counter()
    got = cpu.generate_greedy(res["prompt"], tokens + 1)
    tn = time.perf_counter() - t
    cpu.close()
    d = max(tn - t1, 1e-9)
    return {
        "tok_s": round(tokens / d, 3), "cores": threads, "kind": "port",
        "sample": f"64-token prefill then {tokens} greedy steps, {threads} threads; "
                  f"same tokens as the GPU: {bool(np.array_equal(got[:tokens], res['tokens'][:tokens]))}",
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
    """A short, fixed sequence for `rocprofv3 --pmc` runs: each GEMV workload's
    step on rotating copies, the prefill GEMMs at 512 and 2048 tokens, then
    device-to-device copies of a known size (the calibration for the
    counters)."""
    import rusticide_amd as R
    from rusticide_amd import hip as H
    from rusticide_amd import synth

    ctx = R.Context(0)
    for name in (HEADLINE, "q6k_ffn_down", "q4k_ffn_gate", "i2s_up", "i2s_down"):
        type_id, rows, cols = WORKLOADS[name][:3]
        _, mats = load_rotation(ctx, name)
        x = H.DeviceArray.from_numpy(synth.normal_f32(cols, seed=2))
        out = H.DeviceArray(rows)
        R.matmul_batch_device_repeat(ctx, x, 1, mats, out, steps)
        H.synchronize()
        for m in mats:
            m.free()
        log(f"[pmc] {name}: {steps} steps")
    # the prefill GEMMs, for their MFMA / VALU / LDS counters: Q4_K ffn_gate
    # and Q6_K ffn_down at 512 and 2048 tokens, five launches each, in order
    for type_id, rows, cols in ((12, 5632, 2048), (14, 2048, 5632)):
        m = R.Matrix.load(ctx, type_id, synth.matrix(type_id, rows, cols, seed=1), rows, cols)
        for T in (512, 2048):
            x = H.DeviceArray.from_numpy(synth.normal_f32(T * cols, seed=2))
            out = H.DeviceArray(rows * T)
            q8 = R.Q8(ctx).quantize(x, T, R.SUPER_BLOCK)
            for _ in range(5):
                R.dot_matrix_device(m, q8, out)
            H.synchronize()
            q8.free()
            log(f"[pmc] prefill GEMM type {type_id} {rows}x{cols} x {T} tokens: 5 launches")
        m.free()
    n = 256 * 2 ** 20
    a, b = H.DeviceArray(n // 4), H.DeviceArray(n // 4)
    a.fill_bytes(1)
    for _ in range(3):
        H.check(H.hip().hipMemcpy(b.ptr, a.ptr, n, H.D2D), "hipMemcpy D2D")
    H.synchronize()
    log(f"[pmc] copy: 3 x {n} bytes device to device")
    ctx.close()
    return 0


def pmc_prefill(reps: int) -> int:
    """A short sequence for `rocprofv3 --pmc` runs over the batched forward:
    `reps` 64-token prefills (Decoder.forward_batch from position 0) of the
    e2e section's TinyLlama-shaped model, after one untimed one."""
    import rusticide_amd as R
    from rusticide_amd import hip as H
    from rusticide_amd import synth

    ctx = R.Context(0)
    dec = R.Decoder(ctx, synth.decoder_model(synth.TINYLLAMA, seed=7))
    prompt = np.random.default_rng(1).integers(0, synth.TINYLLAMA["vocab_size"], 64).astype(np.uint32)
    for _ in range(reps + 1):
        dec.reset()
        dec.forward_batch(prompt, 0)
    H.synchronize()
    log(f"[pmc] prefill: {reps + 1} x 64-token forward_batch")
    dec.close()
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
    ap.add_argument("--pmc-prefill", action="store_true", help="run 64-token prefills for rocprofv3 --pmc")
    ap.add_argument("--decode-reps", type=int, default=5, help="timed 64+128-token generations (0 skips)")
    ap.add_argument("--no-gemm", action="store_true", help="skip the prefill GEMM measurement")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU: the path runs on a single MI355X (asked for "
              f"--gpus {args.gpus}, WORLD_SIZE={world}); multi-GPU sharding is design-only.",
              file=sys.stderr)
        return 2
    if args.pmc:
        return pmc_probe(20)
    if args.pmc_prefill:
        return pmc_prefill(5)

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
    # the measured ceiling of each workload: a plain streaming read of the
    # same bytes per launch over the same rotation of copies
    for name, r in results.items():
        r["stream_gbs"] = measure_stream_read(ctx, r["bytes"], r["copies"], args.steps, args.warmup)
        log(f"[bench] {name}: streaming read of the same {r['bytes']:,} bytes per launch "
            f"{r['bytes'] / r['stream_gbs'] / 1e3:.2f} us = {r['stream_gbs']:.0f} GB/s; "
            f"the GEMV kernel reaches {100 * r['kernel_gbs'] / r['stream_gbs']:.1f}% of it")
    stream_gbs = h["stream_gbs"]
    gemm = None if args.no_gemm else measure_gemm(ctx)
    if gemm:
        for g in gemm:
            log(f"[bench] prefill GEMM {g['workload']} x {g['tokens']} tokens: kernel {g['gemm_kernel_us']} us "
                f"({g['kernel_tops']} TOPS, {100 * g['mfma_frac']:.1f}% of int8 peak), step {g['step_us']} us")
    e2e = None
    if args.decode_reps > 0:
        e2e = measure_decode(ctx, args.decode_reps)
        log(f"[bench] e2e decode: {e2e['tok_s']:.1f} tok/s ({e2e['us_per_token']:.1f} us/token, "
            f"{e2e['gbs']:.0f} GB/s of compulsory bytes), prefill 64 tokens {e2e['prefill_ms']:.2f} ms "
                f"(a one-token generation, prefill + pick + the pick's forward: {e2e['generate_1_ms']:.2f} ms)")
    cpu = None if args.no_cpu else measure_cpu(h, args.cpu_seconds)
    if cpu:
        log(f"[bench] cpu baseline: {cpu['value']} GB/s ({cpu['sample']})")
    cpu_decode = None if (args.no_cpu or e2e is None) else measure_cpu_decode(e2e)
    if cpu_decode:
        log(f"[bench] cpu decode: {cpu_decode['tok_s']} tok/s ({cpu_decode['sample']})")
    also = {
        n: {"workload": r["desc"], "step_gbs": round(r["step_gbs"], 1), "kernel_us": round(r["kernel_us"], 3),
            "kernel_gbs": round(r["kernel_gbs"], 1), "hbm_frac": round(r["kernel_gbs"] / HBM_PEAK_GBS, 4),
            "warm_kernel_gbs": round(r["warm_kernel_gbs"], 1), "bytes_per_launch": r["bytes"],
            "stream_read_gbs": round(r["stream_gbs"], 1),
            "frac_of_stream_read": round(r["kernel_gbs"] / r["stream_gbs"], 4),
            "prequantized_gemv_us": round(r["prequantized_gemv_us"], 3),
            "unheld_kernel_us": round(r["unheld_kernel_us"], 3), "warmup_launches": r["warmup_launches"],
            "host_us_per_launch": round(r["host_us_per_launch"], 2), "queued_inside_hold": r["held"],
            "kernel": r["kernel"], "hbm_traffic_bytes": traffic_for(n)}
        for n, r in results.items() if n != HEADLINE
    }
    if gemm is not None:
        also["prefill_gemm"] = {"workload": "int8 MFMA GEMMs x N tokens, bit-identical to the CPU path",
                                "runs": gemm, "peak_tops": INT8_PEAK_TOPS}
    if e2e is not None:
        also["e2e_decode"] = {
            "workload": "TinyLlama-1.1B-shaped Q4_K_M random-init model, 64-token prompt + 128 greedy tokens, "
                        "batch 1, f32 KV cache",
            "tok_s": round(e2e["tok_s"], 1), "us_per_token": round(e2e["us_per_token"], 1),
            "prefill_64_ms": round(e2e["prefill_ms"], 3), "generate_1_ms": round(e2e["generate_1_ms"], 3),
            "bytes_per_token": e2e["bytes_per_token"], "compulsory_gbs": round(e2e["gbs"], 1),
            "hbm_frac": round(e2e["gbs"] / HBM_PEAK_GBS, 4),
            "gguf_load": {k: (round(v, 2) if isinstance(v, float) else v) for k, v in e2e["gguf_load"].items()},
            "cpu_oracle": cpu_decode,
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
                   "warmup_launches": h["warmup_launches"],
                   "step": "one launch: in-workgroup Q8_K quantize + Q6_K GEMV, weights rotated over >1 GiB"},
        "roofline": {"bound": "hbm", "achieved": round(h["kernel_gbs"], 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(h["kernel_gbs"] / HBM_PEAK_GBS, 4),
                     "traffic": traffic_for(HEADLINE),
                     "kernel": h["kernel"], "kernel_avg_us": round(h["kernel_us"], 3),
                     "warm_cache_resident_gbs": round(h["warm_kernel_gbs"], 1),
                     "stream_read_gbs": round(stream_gbs, 1),
                     "frac_of_stream_read": round(h["kernel_gbs"] / stream_gbs, 4),
                     "prequantized_gemv_us": round(h["prequantized_gemv_us"], 3),
                     "unheld_kernel_avg_us": round(h["unheld_kernel_us"], 3),
                     "queued_inside_hold": h["held"],
                     "host_us_per_launch": round(h["host_us_per_launch"], 2),
                     "timing": "HIP events on the kernel's stream around max(steps, 200) launches queued "
                               "behind a bounded hold (back to back); unheld_kernel_avg_us: events around "
                               "the wall-clock timed region itself"},
        "cpu_baseline": cpu,
        "also": also,
    }
    ctx.close()
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
