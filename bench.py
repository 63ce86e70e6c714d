#!/usr/bin/env python3
"""Benchmark of the gfx950 quantized matvec path on one MI355X.

Headline workload: Q4_K decode matvec, 14336 rows x 4096 cols (the Llama-3-8B
FFN gate/up shape), batch 1.  One step = one rlq_matmul, which is one kernel:
it quantizes the fp32 activation to Q8_K in its prologue and runs the
Q4_K x Q8_K matvec.  The metric's second half, the prefill GEMM (M=512 tokens
against the same weights), is reported in the same line under "prefill": one
step = one rlq_matmul with batch 512 (Q8_K quantizer kernel + GEMM kernel).  Weights are N(0, 0.02) fp32 quantized by this library's
own Q4_K encoder on the GPU (bit-exact with the reference's encoder);
activations are N(0, 1) fp32; both are resident in HBM before timing.

Cache honesty: 33 MB of weights fit in the 256 MB MALL, so the timed loop
rotates over ROTATE distinct weight copies (>= 330 MB per sweep).

value     = algorithmic bytes per step (W + fp32 x + fp32 y) / mean step time,
            the K timed steps bracketed by HIP events on the stream they run on
roofline  = the same bytes / the mean step time; the step is one kernel, so
            this is that kernel's mean duration launched back to back (the
            rocprofv3 kernel trace of the same command agrees), against
            MI355X's 8 TB/s HBM peak
cpu_baseline = the CPU oracle (a C restatement of the reference's scalar
            Rust path) on the same weights, 1 thread, repeated for ~10 s.

--copy-probe adds one device-to-device copy of 256 MiB before the timed steps:
the calibration kernel for FETCH_SIZE / WRITE_SIZE counter runs.

"configs" times every other BASELINE configuration the same way, each with its own roofline:
Q8_0 4864x896 (batch 1), Q4_K 14336x4096 at batches 4 and 8, the Q6_K 128256x4096 output
projection at batches 1 and 8 with the fused greedy argmax, and the Qwen-vocabulary output
projection 151936x896 as Q8_0 (Q6_K has no encoding at K=896) with the argmax.  Matrices that fit
the 256 MB MALL rotate over copies so that a sweep touches >= 300 MB.

"prefill" prices the GEMM against the int8 MFMA peak (5.0 POP/s), the figure the target is
quoted on.

"decode_step" (config 5) times whole decode steps of a random-init Llama-3-8B-shape model
(Q4_K layers, Q6_K output) at a context of ~1000 rows: tok/s and the step's algorithmic bytes
(every weight byte once + the KV rows read) per second, with one oracle step on one host thread
as its CPU baseline.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--extra] [--no-cpu] [--copy-probe]
                       [--no-llama] [--no-configs] [--llama-steps N] [--no-llama-cpu]
"""
import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
F16_MFMA_PEAK_TFLOPS = 2500.0  # dense f16 MFMA, the instructions the GEMM issues
INT8_MFMA_PEAK_TOPS = 5000.0   # dense int8 MFMA
ROTATE = 10
PREFILL_M = 512
# HBM bytes per launch of this build's kernels, measured with rocprofv3 --pmc FETCH_SIZE and
# WRITE_SIZE (each calibrated against a 256 MiB device copy), recorded in
# profiles/hbm_traffic_q4k_decode_and_prefill.md: the decode kernel, and the prefill step's
# two kernels (GEMM + quantizer).
TRAFFIC_DECODE_BYTES = 33351490
TRAFFIC_PREFILL_BYTES = 98617131 + 12975038
# the same measurement for the kernels of the other configurations (per launch)
TRAFFIC_CONFIG_BYTES = {
    "q8_0_4864x896_b1": 4961661,
    "q4k_14336x4096_b4": 34064124,
    "q4k_14336x4096_b8": 33980196 + 224233,  # the matvec, then the planes kernel
    "q6k_128256x4096_b1_argmax": 436357969,
    "q6k_128256x4096_b8_argmax": 440944786,
    "q8_0_151936x896_b1_argmax": 146142805,
}
COPY_PROBE_BYTES = 256 << 20
METRIC = "Q4_K matvec GB/s (14336x4096, B=1) + prefill GEMM TOPS (M=512); tok/s"


def load():
    import importlib

    return importlib.import_module("rust-llama_amd")


def gpu_weights(rlq, ctx, dtype, rows, cols, seed, copies):
    """N(0, 0.02) fp32 generated and quantized on the GPU; returns handles
    and the host bytes of copy 0."""
    torch = rlq.torch
    g = torch.Generator(device="cuda")
    handles, host0 = [], None
    for c in range(copies):
        g.manual_seed(seed + 1000 * c)
        xw = torch.randn((rows, cols), generator=g, device="cuda", dtype=torch.float32) * 0.02
        packed = ctx.quantize(dtype, xw)
        ctx.sync()
        del xw
        handles.append(rlq.Weights(ctx, dtype, packed, rows, cols))
        if c == 0:
            host0 = packed.cpu().numpy()
        del packed
    return handles, host0


def algorithmic_bytes(rlq, dtype, rows, cols, batch):
    return rlq.row_bytes(dtype, cols) * rows + 4 * cols * batch + 4 * rows * batch


def time_steps(rlq, ctx, handles, x, y, steps, warmup, argmax=None):
    """Mean step time (ms) of `steps` back-to-back rlq_matmul calls (or
    rlq_matmul_argmax when `argmax` is given) through prepared calls
    (Context.bind_matmul), bracketed by HIP events on the stream they are
    launched on (torch's current one)."""
    torch = rlq.torch
    n = len(handles)
    # prepared calls (tensors, stream and error record resolved once), so the
    # host issues launches faster than the GPU retires them
    bound = [ctx.bind_matmul(h, x, y, argmax) for h in handles]

    def call(i):
        bound[i % n]()

    for i in range(warmup):
        call(i)
    ctx.sync()
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for i in range(steps):
        call(i)
    end.record(stream)
    torch.cuda.synchronize()
    ctx.sync()  # raises if the GPU recorded a data error
    return start.elapsed_time(end) / steps


def call_distribution(rlq, ctx, handles, x, y, calls):
    """Median and p90 of single rlq_matmul calls, each bracketed by its own
    pair of HIP events on the launch stream (weights rotated as in the timed
    loop); the events' own cost is included."""
    torch = rlq.torch
    n = len(handles)
    stream = torch.cuda.current_stream()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(calls)]
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(ev):
        a.record(stream)
        ctx.matmul(handles[i % n], x, y)
        b.record(stream)
    torch.cuda.synchronize()
    ctx.sync()
    us = np.sort(np.array([a.elapsed_time(b) * 1e3 for a, b in ev]))
    return {"calls": calls, "median_us": round(float(np.median(us)), 3),
            "p90_us": round(float(us[int(0.9 * (calls - 1))]), 3)}


def practical_peaks(torch, rlq=None, reps=20):
    """Measured ceilings beside the spec peaks: a 1 GiB device-to-device copy
    (bytes read + written per second), torch's (hipBLASLt) dense f16 and int8
    GEMMs at 8192^3 and at the prefill shape 512x4096x14336, and the library's
    probes: chained MFMAs from registers (v_mfma_i32_32x32x32_i8 and
    v_mfma_f32_32x32x16_f16), LDS reads in the prefill GEMM's A-operand
    pattern alone and feeding f16 MFMAs at the GEMM's ratio, and a plain read
    of the headline's weight bytes with the one-column matvec's launch shape
    and loads, over the same 10 rotated copies (rlq_probe_mfma,
    rlq_probe_stream)."""
    out = {}

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            fn()
        b.record()
        torch.cuda.synchronize()
        return a.elapsed_time(b) / reps * 1e-3

    src = torch.empty(1 << 30, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    out["copy_gbs"] = round(2 * src.numel() / timed(lambda: dst.copy_(src)) / 1e9, 1)
    del src, dst
    n = 8192
    a = torch.randn((n, n), device="cuda", dtype=torch.float16)
    b = torch.randn((n, n), device="cuda", dtype=torch.float16)
    out["f16_gemm_tflops"] = round(2 * n ** 3 / timed(lambda: torch.mm(a, b)) / 1e12, 1)
    del a, b
    try:
        a8 = torch.randint(-127, 127, (n, n), device="cuda", dtype=torch.int8)
        b8 = torch.randint(-127, 127, (n, n), device="cuda", dtype=torch.int8)
        out["int8_gemm_tops"] = round(2 * n ** 3 / timed(lambda: torch._int_mm(a8, b8)) / 1e12, 1)
        del a8, b8
    except (RuntimeError, AttributeError) as e:
        out["int8_gemm_tops"] = None
        out["int8_note"] = str(e).splitlines()[0][:120]
    # the same library GEMMs at the prefill shape (M=512 tokens, K=4096, N=14336):
    # the ceiling a dense, unquantized product of that shape reaches here
    m, k, nn = PREFILL_M, 4096, 14336
    a = torch.randn((m, k), device="cuda", dtype=torch.float16)
    b = torch.randn((k, nn), device="cuda", dtype=torch.float16)
    out["f16_gemm_prefill_shape_tflops"] = round(2 * m * k * nn / timed(lambda: torch.mm(a, b)) / 1e12, 1)
    del a, b
    try:
        a8 = torch.randint(-127, 127, (m, k), device="cuda", dtype=torch.int8)
        b8 = torch.randint(-127, 127, (k, nn), device="cuda", dtype=torch.int8)
        out["int8_gemm_prefill_shape_tops"] = round(2 * m * k * nn / timed(lambda: torch._int_mm(a8, b8)) / 1e12, 1)
        del a8, b8
    except (RuntimeError, AttributeError) as e:
        out["int8_gemm_prefill_shape_tops"] = None
        out["int8_prefill_note"] = str(e).splitlines()[0][:120]
    if rlq is not None:
        out.update(probe_peaks(rlq, torch, reps))
    torch.cuda.empty_cache()
    return out


def probe_peaks(rlq, torch, reps):
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    stream = torch.cuda.current_stream()
    sp = ctypes.c_void_p(stream.cuda_stream)
    out = {}
    iters = 4000
    sink = torch.zeros(16 * 4 * cus, dtype=torch.int32, device="cuda")
    # (kind, key, work per wave step, workgroups): the MFMA chains at four
    # workgroups per CU; the LDS reads and the GEMM's ratio at two, the
    # prefill GEMM's occupancy (work per step: 4 MFMAs, or 4 KB read)
    for kind, key, per, wgs in ((0, "mfma_i8_32x32x32_tops", 4 * 2 * 32 * 32 * 32, 4 * cus),
                                (1, "mfma_f16_32x32x16_tflops", 4 * 2 * 32 * 32 * 16, 4 * cus),
                                (2, "lds_read_b128_tbs", 4 * 1024, 2 * cus),
                                (3, "mfma_f16_with_lds_a_reads_tflops", 4 * 2 * 32 * 32 * 16, 2 * cus)):
        def launch():
            rc = rlq._lib.rlq_probe_mfma(kind, wgs, iters, ctypes.c_void_p(sink.data_ptr()), sp)
            if rc != 0:
                raise RuntimeError(f"rlq_probe_mfma: {rc}")
        launch()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(reps):
            launch()
        b.record(stream)
        torch.cuda.synchronize()
        s = a.elapsed_time(b) / reps * 1e-3
        out[key] = round(wgs * 4 * iters * per / s / 1e12, 1)
    # MFMA waves and FMA waves on the same SIMDs (one 8-wave workgroup per CU):
    # each half alone, and together with the MFMA accumulators in VGPRs and in
    # AGPRs.  overlap = the time the pair saves against running the halves one
    # after the other, as a fraction of the shorter half (1: fully hidden)
    co = {}
    for kind, key in ((4, "mfma_alone_us"), (5, "fma_alone_us"), (6, "together_vgpr_acc_us"),
                      (7, "mfma_alone_agpr_acc_us"), (8, "together_agpr_acc_us")):
        def launch():
            rc = rlq._lib.rlq_probe_mfma(kind, cus, 2000, ctypes.c_void_p(sink.data_ptr()), sp)
            if rc != 0:
                raise RuntimeError(f"rlq_probe_mfma: {rc}")
        launch()
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(reps):
            launch()
        b.record(stream)
        torch.cuda.synchronize()
        co[key] = round(a.elapsed_time(b) / reps * 1e3, 1)
    for acc, m in (("vgpr", co["mfma_alone_us"]), ("agpr", co["mfma_alone_agpr_acc_us"])):
        f = co["fma_alone_us"]
        co[f"overlap_{acc}_acc"] = round((m + f - co[f"together_{acc}_acc_us"]) / min(m, f), 2)
    out["mfma_fma_coexec"] = co
    # the headline's bytes (Q4_K 14336x4096: 33,030,144 B) in 10 rotated copies
    nbytes, copies = 14336 * 2304, ROTATE
    bufs = [torch.empty(nbytes, dtype=torch.uint8, device="cuda") for _ in range(copies)]

    def read(i):
        rc = rlq._lib.rlq_probe_stream(ctypes.c_void_p(bufs[i % copies].data_ptr()), nbytes, cus,
                                       ctypes.c_void_p(sink.data_ptr()), sp)
        if rc != 0:
            raise RuntimeError(f"rlq_probe_stream: {rc}")

    for i in range(50):
        read(i)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    n = 2000
    a.record(stream)
    for i in range(n):
        read(i)
    b.record(stream)
    torch.cuda.synchronize()
    us = a.elapsed_time(b) / n * 1e3
    out["stream_floor"] = {"bytes": nbytes, "us_per_pass": round(us, 3), "gbs": round(nbytes / us / 1e3, 1),
                           "note": "33,030,144 weight bytes read with the one-column matvec's grid (one workgroup "
                                   "of 16 waves per CU) and 1 KB non-temporal load runs, 10 rotated copies, "
                                   "launched back to back"}
    # the same bytes read with other launch shapes: waves per workgroup, 1 KB
    # runs in flight per wave, workgroups per CU, non-temporal or plain loads
    sweep = {}
    for waves, runs, per_cu, nt in ((16, 1, 1, 1), (16, 2, 1, 1), (16, 4, 1, 1), (16, 8, 1, 1), (16, 2, 1, 0),
                                    (8, 2, 2, 1), (8, 4, 2, 1), (8, 4, 4, 1), (4, 4, 4, 1), (4, 8, 4, 1),
                                    (4, 4, 8, 1)):
        def read_shape(i):
            rc = rlq._lib.rlq_probe_stream_shape(ctypes.c_void_p(bufs[i % copies].data_ptr()), nbytes, per_cu * cus,
                                                 waves, runs, nt, ctypes.c_void_p(sink.data_ptr()), sp)
            if rc != 0:
                raise RuntimeError(f"rlq_probe_stream_shape: {rc}")

        for i in range(30):
            read_shape(i)
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        n = 500
        a.record(stream)
        for i in range(n):
            read_shape(i)
        b.record(stream)
        torch.cuda.synchronize()
        sweep[f"{waves}w_{runs}r_{per_cu}wg_{'nt' if nt else 'plain'}"] = round(a.elapsed_time(b) / n * 1e3, 3)
    best = min(sweep, key=sweep.get)
    out["stream_shapes_us"] = {"passes": sweep, "best": best,
                               "note": "the stream floor's bytes read with other launch shapes (waves per workgroup, "
                                       "1 KB runs in flight per wave, workgroups per CU, load kind)"}
    del bufs
    return out


def prefill(rlq, ctx, handles, rows, cols, steps, warmup):
    """The prefill GEMM over the rotated weight copies: M=512 tokens of N(0,1)."""
    torch = rlq.torch
    g = torch.Generator(device="cuda")
    g.manual_seed(0x51A7E003)
    x = torch.randn((PREFILL_M, cols), generator=g, device="cuda", dtype=torch.float32)
    y = torch.empty((PREFILL_M, rows), device="cuda", dtype=torch.float32)
    ms = time_steps(rlq, ctx, handles, x, y, steps, warmup)
    ops = 2.0 * PREFILL_M * rows * cols
    tops = ops / (ms * 1e-3) / 1e12
    return {
        "workload": f"Q4_K x Q8_K prefill GEMM, M={PREFILL_M} tokens x K={cols} x N={rows} (Q8_K quantizer "
                    "kernel + GEMM kernel per step)",
        "steps": steps, "us_per_step": round(ms * 1e3, 3), "tops": round(tops, 2),
        "tok_s": round(PREFILL_M / (ms * 1e-3), 1), "ops_per_step": ops,
        "roofline": {"bound": "mfma", "achieved": round(tops, 2), "peak": INT8_MFMA_PEAK_TOPS,
                     "unit": "TOP/s", "frac": round(tops / INT8_MFMA_PEAK_TOPS, 4),
                     "frac_of_f16_peak": round(tops / F16_MFMA_PEAK_TFLOPS, 4),
                     "traffic": TRAFFIC_PREFILL_BYTES},
    }


def host_cpu():
    """The host CPU the CPU baselines ran on: its model name and logical CPU count."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return f"{model}, {os.cpu_count() or 0} logical CPUs visible"


def cpu_baseline(dtype, w_host, rows, cols, x_host, budget_s=10.0, all_cores_s=5.0):
    """Oracle matvec (the reference's scalar path restated in C): 1 thread (the
    reference never threads a matvec), then row-parallel over the host cores
    this job may use (at most 16) as a second figure."""
    import oracle

    def timed(threads, budget):
        t0 = time.perf_counter()
        reps = 0
        while True:
            oracle.matvec(int(dtype), w_host, rows, cols, x_host, threads=threads)
            reps += 1
            el = time.perf_counter() - t0
            if el >= budget:
                return reps, el

    nbytes = w_host.size + 4 * cols + 4 * rows
    reps, el = timed(1, budget_s)
    per = el / reps
    out = {"value": round(nbytes / per / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
           "sample": f"{reps} full {rows}x{cols} Q4_K matvecs of the benchmark's weights in {el:.1f} s "
                     f"({per * 1e3:.1f} ms each), oracle/rlq_oracle.c built with gcc -O2 -ffp-contract=off",
           "host": host_cpu()}
    cores = max(1, min(16, os.cpu_count() or 1))
    if cores > 1:
        reps, el = timed(cores, all_cores_s)
        out["all_cores"] = {"value": round(nbytes / (el / reps) / 1e9, 4), "unit": "GB/s", "cores": cores,
                            "sample": f"{reps} matvecs in {el:.1f} s, rows split over {cores} threads"}
    return out


def run_config(rlq, ctx, dtype, rows, cols, batch, seed, steps, warmup, copies, argmax=False):
    torch = rlq.torch
    handles, host0 = gpu_weights(rlq, ctx, dtype, rows, cols, seed, copies)
    g = torch.Generator(device="cuda")
    g.manual_seed(seed + 7)
    x = torch.randn((batch, cols), generator=g, device="cuda", dtype=torch.float32)
    y = torch.empty((batch, rows), device="cuda", dtype=torch.float32)
    am = torch.empty(batch, device="cuda", dtype=torch.int32) if argmax else None
    ms = time_steps(rlq, ctx, handles, x, y, steps, warmup, argmax=am)
    nbytes = algorithmic_bytes(rlq, dtype, rows, cols, batch) + (4 * batch if argmax else 0)
    out = {"rows": rows, "cols": cols, "batch": batch, "dtype": rlq.DType(dtype).name, "bytes_per_step": nbytes,
           "us_per_step": ms * 1e3, "gbs": nbytes / (ms * 1e-3) / 1e9, "rotated_copies": copies}
    out["frac_hbm"] = out["gbs"] / HBM_PEAK_GBS
    return out, handles, host0, x


# The other BASELINE configurations (name: dtype, rows, cols, batch, rotated copies, fused argmax,
# workload).  Copies bring each timed sweep to >= 300 MB where one matrix fits the MALL.
CONFIGS = {
    "q8_0_4864x896_b1": ("Q8_0", 4864, 896, 1, 64, False,
                         "Q8_0 x Q8_0 decode matvec 4864x896 (Qwen2.5-0.5B FFN up), batch 1"),
    "q4k_14336x4096_b4": ("Q4_K", 14336, 4096, 4, ROTATE, False, "Q4_K x Q8_K decode matvec 14336x4096, batch 4"),
    "q4k_14336x4096_b8": ("Q4_K", 14336, 4096, 8, ROTATE, False, "Q4_K x Q8_K decode matvec 14336x4096, batch 8"),
    "q6k_128256x4096_b1_argmax": ("Q6_K", 128256, 4096, 1, 1, True,
                                  "Q6_K output projection 128256x4096, batch 1, fused greedy argmax"),
    "q6k_128256x4096_b8_argmax": ("Q6_K", 128256, 4096, 8, 1, True,
                                  "Q6_K output projection 128256x4096, batch 8, fused greedy argmax"),
    "q8_0_151936x896_b1_argmax": ("Q8_0", 151936, 896, 1, 3, True,
                                  "Qwen-vocabulary output projection 151936x896 as Q8_0 (Q6_K cannot encode "
                                  "K=896), batch 1, fused greedy argmax"),
}


def config_legs(rlq, ctx, steps, warmup):
    legs = {}
    for i, (name, (dt, r, c, b, copies, am, workload)) in enumerate(CONFIGS.items()):
        o, hs, _, _ = run_config(rlq, ctx, rlq.DType[dt], r, c, b, 0x51A7E010 + i, steps, warmup, copies, argmax=am)
        for h in hs:
            h.close()
        rlq.torch.cuda.empty_cache()
        legs[name] = {"workload": workload, "us_per_step": round(o["us_per_step"], 3),
                      "bytes_per_step": o["bytes_per_step"], "rotated_copies": copies,
                      "roofline": {"bound": "hbm", "achieved": round(o["gbs"], 2), "peak": HBM_PEAK_GBS,
                                   "unit": "GB/s", "frac": round(o["gbs"] / HBM_PEAK_GBS, 4),
                                   "traffic": TRAFFIC_CONFIG_BYTES.get(name)}}
    return legs


def moe_decode(rlq, ctx, steps, warmup):
    """MUL_MAT_ID at a Mixtral-8x7B FFN shape: 8 Q4_K experts of 14336x4096,
    one token routed to 2 of them per step (one activation column shared by
    both slots); the expert pair rotates over 4 disjoint pairs, so the 264 MB
    of experts cannot sit in the 256 MB MALL.  One step = one launch over both
    (token, slot) pairs, each workgroup checking the ids and quantizing the
    column to Q8_K in its prologue."""
    torch = rlq.torch
    DT = rlq.DType
    experts, rows, cols, slots = 8, 14336, 4096, 2
    g = torch.Generator(device="cuda")
    g.manual_seed(0x51A7E00E)
    xw = torch.randn((experts * rows, cols), generator=g, device="cuda", dtype=torch.float32) * 0.02
    packed = ctx.quantize(DT.Q4_K, xw)
    ctx.sync()
    del xw
    W = rlq.Weights(ctx, DT.Q4_K, packed, rows, cols, experts)
    del packed
    x = torch.randn((1, 1, cols), generator=g, device="cuda", dtype=torch.float32)
    ids = [torch.tensor([[2 * i, 2 * i + 1]], dtype=torch.int32, device="cuda") for i in range(4)]
    y = torch.empty((1, slots, rows), device="cuda", dtype=torch.float32)
    for i in range(warmup):
        ctx.mul_mat_id(W, x, ids[i % 4], y=y)
    ctx.sync()
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for i in range(steps):
        ctx.mul_mat_id(W, x, ids[i % 4], y=y)
    end.record(stream)
    torch.cuda.synchronize()
    ctx.sync()
    ms = start.elapsed_time(end) / steps
    nbytes = slots * rlq.row_bytes(DT.Q4_K, cols) * rows + 4 * cols + 4 * slots * rows + 8
    W.close()
    return {"workload": "MUL_MAT_ID Q4_K, 8 experts of 14336x4096, 1 token, top-2 (one launch per step: id "
                        "check, Q8_K quantizer and both experts' matvecs)",
            "steps": steps, "us_per_step": round(ms * 1e3, 3), "bytes_per_step": nbytes,
            "gbs": round(nbytes / (ms * 1e-3) / 1e9, 2), "frac_hbm": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}


# Llama-3-8B decode-step shape: 32 layers, d_model 4096, 32 query / 8 KV heads of 128, FFN 14336,
# vocabulary 128256, f32 KV cache of 1024 rows; Q4_K layer matrices and embedding, Q6_K output.
LLAMA = dict(vocabulary=128256, width=4096, feed_forward=14336, heads=32, kv_heads=8, max_context=1024,
             n_layers=32, rms_epsilon=1e-5, rope_base=500000.0)


def q4km_more(i, n):
    """The layers whose attn_v and ffn_down a Q4_K_M file stores in Q6_K: the first and last eighth
    and every third layer between (crates/model-quant/src/planner.rs:221-223, 346, 391-402)."""
    return i < n // 8 or i >= 7 * n // 8 or (i - n // 8) % 3 == 2


def llama_tensors(rlq, ctx, cfg, seed, q4km=False):
    """Random-init weights on the GPU: matrices N(0, 0.02) and the embedding N(0, 1) in f32, encoded
    by the library's own Q4_K / Q6_K encoders; norm weights N(1, 0.05).  q4km: the value and down
    matrices of the q4km_more layers in Q6_K (the layer's `types`), as in a Q4_K_M file."""
    torch = rlq.torch
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    DT = rlq.DType

    def mat(dtype, rows, cols, std=0.02):
        x = torch.randn((rows, cols), generator=g, device="cuda", dtype=torch.float32) * std
        out = ctx.quantize(dtype, x)
        del x
        return out

    def norm(n):
        return torch.randn(n, generator=g, device="cuda", dtype=torch.float32) * 0.05 + 1.0

    W, F, kvw = cfg.width, cfg.feed_forward, cfg.kv_width
    layers = []
    for i in range(cfg.n_layers):
        vd = DT.Q6_K if q4km and q4km_more(i, cfg.n_layers) else DT.Q4_K
        layer = {"attention_norm": norm(W), "query": mat(DT.Q4_K, W, W), "key": mat(DT.Q4_K, kvw, W),
                 "value": mat(vd, kvw, W), "attention_output": mat(DT.Q4_K, W, W),
                 "feed_forward_norm": norm(W), "gate": mat(DT.Q4_K, F, W), "up": mat(DT.Q4_K, F, W),
                 "down": mat(vd, W, F)}
        if vd != DT.Q4_K:
            layer["types"] = {"value": int(vd), "down": int(vd)}
        layers.append(layer)
    emb = torch.cat([mat(DT.Q4_K, 8016, W, 1.0) for _ in range(cfg.vocabulary // 8016)])
    t = {"embedding": emb, "output_norm": norm(W), "output": mat(DT.Q6_K, cfg.vocabulary, W), "layers": layers}
    ctx.sync()
    return t


def decode_step(rlq, ctx, steps, warmup, cpu=False, q4km=False):
    """Config 5: one decode step of the Llama-3-8B-shape model per token (embedding row, 32 layers,
    final norm, Q6_K output matvec, greedy argmax), with synthetic tokens.  The random-init model is
    written as a GGUF file by the library's GGUF writer and loaded by its llama GGUF loader
    (rlq_llama_create_from_gguf); the KV cache is filled to max_context - warmup - steps rows
    first, so the timed steps see a context of ~1000 rows."""
    import shutil
    import tempfile

    torch = rlq.torch
    DT = rlq.DType
    L = LLAMA
    cfg = rlq.LlamaConfig(L["vocabulary"], L["width"], L["feed_forward"], L["heads"], L["kv_heads"],
                          L["max_context"], L["n_layers"], L["rms_epsilon"], L["rope_base"], 0.0, DT.Q4_K, DT.Q6_K,
                          DT.Q4_K)
    t0 = time.perf_counter()
    tensors = llama_tensors(rlq, ctx, cfg, 0x51A7E005, q4km=q4km)
    gen_s = time.perf_counter() - t0
    host_tensors = {"embedding": tensors["embedding"].cpu().numpy(),
                    "output_norm": tensors["output_norm"].cpu().numpy(),
                    "output": tensors["output"].cpu().numpy(),
                    "layers": [{k: (v if k == "types" else v.cpu().numpy()) for k, v in l.items()}
                               for l in tensors["layers"]]}
    n_q6 = sum(1 for l in host_tensors["layers"] if "types" in l)
    del tensors
    torch.cuda.empty_cache()
    tmp = tempfile.mkdtemp(prefix="rlq-llama-")
    try:
        path = os.path.join(tmp, "llama3-8b-shape-q4k.gguf")
        t0 = time.perf_counter()
        rlq.write_llama_gguf(path, cfg, host_tensors)
        write_s = time.perf_counter() - t0
        file_bytes = os.path.getsize(path)
        t0 = time.perf_counter()
        model = rlq.LlamaModel.from_gguf(ctx, path, cfg.max_context)
        load_s = time.perf_counter() - t0
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    if not cpu:
        host_tensors = None
    rng = np.random.default_rng(5)
    toks = rng.integers(0, cfg.vocabulary, size=cfg.max_context).tolist()
    h = torch.empty(cfg.width, dtype=torch.float32, device="cuda")
    am = torch.empty(1, dtype=torch.int32, device="cuda")
    fill = cfg.max_context - warmup - steps
    if fill < 0:
        raise ValueError("warmup + steps exceed the 1024-row context")

    def one(pos):
        model.embedding(toks[pos], h)
        model.step(h, pos, embedding=False, logits=False, argmax=True)

    for pos in range(fill + warmup):
        one(pos)
    ctx.sync()
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for pos in range(fill + warmup, fill + warmup + steps):
        one(pos)
    end.record(stream)
    torch.cuda.synchronize()
    ctx.sync()
    ms = start.elapsed_time(end) / steps
    kvw = cfg.kv_heads * (cfg.width // cfg.heads)
    def layer_bytes(vd):
        return rlq.row_bytes(DT.Q4_K, cfg.width) * (2 * cfg.width + kvw + 2 * cfg.feed_forward) \
            + rlq.row_bytes(vd, cfg.width) * kvw + rlq.row_bytes(vd, cfg.feed_forward) * cfg.width

    weights = (cfg.n_layers - n_q6) * layer_bytes(DT.Q4_K) + n_q6 * layer_bytes(DT.Q6_K) \
        + rlq.row_bytes(DT.Q6_K, cfg.width) * cfg.vocabulary
    mean_ctx = fill + warmup + (steps + 1) / 2.0
    kv = 2 * cfg.n_layers * mean_ctx * kvw * 4
    nbytes = weights + kv
    gbs = nbytes / (ms * 1e-3) / 1e9
    out = {"workload": "Llama-3-8B-shape decode step: 32 layers, d 4096, 32/8 heads of 128, FFN 14336, vocab 128256, "
                       + ("Q4_K_M layout (attn_v and ffn_down of %d layers in Q6_K, the rest Q4_K)" % n_q6
                          if q4km else "Q4_K layers") + " + Q6_K output, f32 KV cache; embedding row + 32 layers + "
                       "final norm + output matvec + greedy argmax per token",
           "steps": steps, "context_rows": [fill + warmup + 1, fill + warmup + steps],
           "ms_per_token": round(ms, 4), "tok_s": round(1e3 / ms, 2),
           "bytes_per_token": int(nbytes), "weight_bytes": int(weights), "kv_bytes_mean": int(kv),
           "achieved_gbs": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
           "data": "synthetic random-init weights (N(0,0.02) matrices, N(0,1) embedding, N(1,0.05) norms) and "
                   "random tokens", "weight_generation_s": round(gen_s, 1),
           "gguf": {"file_bytes": file_bytes, "write_s": round(write_s, 2), "load_s": round(load_s, 2),
                    "how": "written by rlq_gguf_write (the library's GGUF v3 writer), loaded by "
                           "rlq_llama_create_from_gguf"}}
    if cpu:
        import oracle

        oc = type("C", (), {})()
        for k, v in L.items():
            setattr(oc, k, v)
        oc.attention_scale, oc.weight_type, oc.output_type, oc.embedding_type = 0.0, 12, 14, 12
        orc = oracle.LlamaOracle(oc, host_tensors, threads=1)
        # the same work as a GPU step: a context of ~1000 rows (the cache
        # filled with N(0, 1) rows; attention reads every row the step sees)
        pos = int(round(mean_ctx)) - 1
        crng = np.random.default_rng(6)
        orc.k_cache[:, :pos] = crng.standard_normal((orc.k_cache.shape[0], pos, orc.k_cache.shape[2]),
                                                    dtype=np.float32)
        orc.v_cache[:, :pos] = crng.standard_normal((orc.v_cache.shape[0], pos, orc.v_cache.shape[2]),
                                                    dtype=np.float32)
        orc.cached = pos
        x = orc.embedding(toks[pos])
        t1 = time.perf_counter()
        orc.step(x, pos)
        el = time.perf_counter() - t1
        out["cpu_baseline"] = {"value": round(1.0 / el, 4), "unit": "tok/s", "cores": 1, "kind": "port",
                               "sample": f"one decode step at context {pos + 1} (the oracle's scalar restatement, "
                                         f"1 thread; the KV cache pre-filled with N(0,1) rows): {el:.2f} s",
                               "host": host_cpu()}
    model.close()
    torch.cuda.empty_cache()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--extra", action="store_true", help="also time the other decode configs")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-probe", action="store_true", help="one 256 MiB device copy (counter calibration)")
    ap.add_argument("--no-llama", action="store_true", help="skip the Llama decode step (config 5)")
    ap.add_argument("--llama-steps", type=int, default=32)
    ap.add_argument("--no-llama-cpu", action="store_true", help="skip the oracle decode step on the host")
    ap.add_argument("--no-configs", action="store_true", help="skip the other BASELINE configurations")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one MI355X: every GPU box here has one GPU and this build has no "
              "multi-GPU path (run with --gpus 1)", file=sys.stderr)
        sys.exit(2)

    rlq = load()
    torch = rlq.torch
    DT = rlq.DType
    torch.cuda.set_device(0)
    ctx = rlq.Context(0)

    if args.copy_probe:
        src = torch.empty(COPY_PROBE_BYTES, dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    rows, cols = 14336, 4096
    head, handles, host0, x = run_config(rlq, ctx, DT.Q4_K, rows, cols, 1, 0x51A7E002, args.steps, args.warmup,
                                         ROTATE)
    result = {
        "metric": METRIC,
        "value": round(head["gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["us_per_step"] / 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic: N(0,0.02) fp32 weights quantized to Q4_K on the GPU; N(0,1) fp32 activations",
        "config": {"workload": "Q4_K x Q8_K decode matvec 14336x4096, batch 1 (fused Q8_K quantize + matvec "
                               "per step, one kernel)",
                   "rows": rows, "cols": cols, "batch": 1, "rotated_weight_copies": ROTATE,
                   "bytes_per_step": head["bytes_per_step"]},
        "roofline": {"bound": "hbm", "achieved": round(head["gbs"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(head["gbs"] / HBM_PEAK_GBS, 4), "traffic": TRAFFIC_DECODE_BYTES},
    }
    y1 = torch.empty((1, rows), device="cuda", dtype=torch.float32)
    result["single_call"] = call_distribution(rlq, ctx, handles, x, y1, 200)
    # secondary: one weight copy, left resident in the 256 MB MALL between calls
    warm_ms = time_steps(rlq, ctx, handles[:1], x, y1, args.steps, args.warmup)
    result["warm"] = {"us_per_step": round(warm_ms * 1e3, 3),
                      "gbs": round(head["bytes_per_step"] / (warm_ms * 1e-3) / 1e9, 2),
                      "note": "the same call on one weight copy (cache-resident); the headline rotates 10 copies"}
    result["prefill"] = prefill(rlq, ctx, handles, rows, cols, max(50, args.steps // 10), max(5, args.warmup // 5))
    result["practical_peaks"] = practical_peaks(torch, rlq)
    if not args.no_cpu:
        xh = x.cpu().numpy().reshape(-1)
        result["cpu_baseline"] = cpu_baseline(DT.Q4_K, host0, rows, cols, xh)
    for h in handles:
        h.close()
    torch.cuda.empty_cache()
    if not args.no_configs:
        result["configs"] = config_legs(rlq, ctx, max(200, args.steps // 4), args.warmup)
    if not args.no_llama:
        result["decode_step"] = decode_step(rlq, ctx, args.llama_steps, 8, cpu=not (args.no_llama_cpu or args.no_cpu))
    if args.extra:
        extra = {}
        for name, (t, r, c, b, copies) in {
            "q5k_14336x4096_b1": (DT.Q5_K, 14336, 4096, 1, ROTATE),
            "q5k_14336x4096_b8": (DT.Q5_K, 14336, 4096, 8, ROTATE),
            "q3k_14336x4096_b1": (DT.Q3_K, 14336, 4096, 1, ROTATE),
            "q3k_14336x4096_b8": (DT.Q3_K, 14336, 4096, 8, ROTATE),
            "q2k_14336x4096_b1": (DT.Q2_K, 14336, 4096, 1, ROTATE),
            "q2k_14336x4096_b8": (DT.Q2_K, 14336, 4096, 8, ROTATE),
            # the Q6_K matrices of a Q4_K_M file below the output head: ffn_down, attn_v
            "q6k_4096x14336_b1": (DT.Q6_K, 4096, 14336, 1, ROTATE),
            "q6k_1024x4096_b1": (DT.Q6_K, 1024, 4096, 1, 9 * ROTATE),  # 3.4 MB: 310 MB over the copies
        }.items():
            o, hs, _, _ = run_config(rlq, ctx, t, r, c, b, 0x51A7E000 + len(extra), max(200, args.steps // 4),
                                     args.warmup, copies)
            for h in hs:
                h.close()
            extra[name] = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in o.items()}
            torch.cuda.empty_cache()
        extra["moe_q4k_8x14336x4096_top2"] = moe_decode(rlq, ctx, max(200, args.steps // 4), args.warmup)
        torch.cuda.empty_cache()
        extra["decode_step_q4km"] = decode_step(rlq, ctx, args.llama_steps, 8, cpu=False, q4km=True)
        result["extra"] = extra
    ctx.close()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
