#!/usr/bin/env python3
"""Benchmark of the MI355X TinyTensor attention path (one GPU).

Headline workload (configuration c5, the MFMA-utilisation
config): causal attention forward + backward, bf16 inputs with fp32
accumulation, B=4, H=32, L=4096, d=128.  One step = one forward
(``tt_attn_fwd_bf16``) plus one backward (``tt_attn_bwd_bf16``) over inputs
already resident in HBM.  ``value`` is the algorithmic rate in TFLOP/s:
fwd = 4*B*H*L^2*d, bwd = 8*B*H*L^2*d (dV, dP, dQ, dK; recompute not counted),
both halved by the causal mask -> 1.6493e12 FLOP per step.

Second line item (``decode``): single-query decode, B=64, H=32, Lkv=8192,
d=128, bf16, judged on HBM GB/s over K + V + q + o = 8,590,983,168 bytes.

Per-kernel times come from HIP events recorded on the library stream right
after each kernel launch (``tt_set_launch_events``) inside the timed region;
``roofline`` is reported for the kernel with the largest share of the step.

``cpu_baseline``: the reference's CPU path -- its op chain (Q @ K^T, * s,
+ mask, softmax by max/exp/sum/divide, @ V, and the backward by the same
gradient rules) restated in float32 numpy by ``oracle/attn_oracle.py`` --
timed on a bounded sample of the same workload's heads on the host cores.

Prints ONE JSON line.  ``--gpus N`` with N > 1 exits: this build runs on one
GPU (the (b, h) heads shard across GPUs with no exchange, so N GPUs would run
N independent shares of the same kernels).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "pku-aiprogramming_amd"))

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E

C5 = dict(B=4, H=32, L=4096, d=128)
C4 = dict(B=64, H=32, Lkv=8192, d=128)


# HBM bytes per launch measured by two rocprofv3 PMC runs (FETCH_SIZE, then
# WRITE_SIZE), scaled by a 1 GiB copy kernel's readings (fetch x2.000,
# write x1.000); the commands and raw counters are in
# profiles/hbm_traffic_c5_c4.md.  Re-measured whenever a kernel changes.
MEASURED_TRAFFIC_MIB = {
    "attn_fwd": 555.8,
    "attn_bwd_dq": 883.8,      # also the row pre-pass: reads O, writes -D and LSE log2(e)
    "attn_bwd_dkdv": 1020.1,   # the persistent 256-key kernel at d = 128
    "attn_decode_split": 8193.2,
    "softmax_reg": 2048.1,      # k_softmax_reg<16>, 262144 x 1024 fp32 (profiles/softmax_rows_kernel_stats.md)
    "gemm_bf16_nn": 2527.8 + 149.6,  # k_gemm_dma 8192^3 NN (profiles/gemm_kernel_stats.md)
}


def traffic_bytes(kernel):
    mib = MEASURED_TRAFFIC_MIB.get(kernel)
    return None if mib is None else mib * 2 ** 20


def fwdbwd_flops(B, H, L, d, causal=True):
    f = 12.0 * B * H * L * L * d
    return f / 2 if causal else f


def kernel_flops(B, H, L, d):
    """Algorithmic FLOPs each kernel of the step is charged with (causal)."""
    u = 2.0 * B * H * L * L * d / 2  # one L x L x d GEMM under the causal mask
    return {"attn_fwd": 2 * u, "attn_bwd_dq": 1 * u, "attn_bwd_dkdv": 3 * u}


def decode_bytes(B, H, Lkv, d):
    return 2 * (B * H * Lkv * d * 2) + 2 * (B * H * d * 2)


# Untimed run-in before every GPU measurement.  The GPU lowers its clock while
# it idles (between workloads, while a CPU baseline runs) and needs tens of
# milliseconds of load to come back to the steady clock it holds at the
# board's power limit; a few warm-up steps of a short workload end inside that
# ramp (c3 measured 0.25-0.27 ms per step right after idle against 0.214 ms
# steady).  So each workload first runs for PREWARM_S seconds, then its
# `warmup` steps, then the timed steps.
PREWARM_S = 0.3


def prewarm(T, step, seconds=PREWARM_S):
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for _ in range(10):
            step()
        T.lib().sync()


def run_fwdbwd(T, steps, warmup):
    B, H, L, d = C5["B"], C5["H"], C5["L"], C5["d"]
    scale = float(__import__("numpy").float32(1.0 / math.sqrt(d)))
    shp = (B, H, L, d)
    q, k, v, do = (T.DeviceBuffer(shp, "bf16") for _ in range(4))
    for i, b in enumerate((q, k, v, do)):
        b.fill_normal(5000 + i)
    o, dq, dk, dv = (T.DeviceBuffer(shp, "bf16") for _ in range(4))
    lse = T.DeviceBuffer((B, H, L), "f32")

    def step():
        T.attn_fwd(q, k, v, o, lse, scale, True)
        T.attn_bwd(q, k, v, o, lse, do, dq, dk, dv, scale, True)

    prewarm(T, step)
    for _ in range(warmup):
        step()
    T.lib().sync()

    # launch order of one step: the forward, then the backward's dQ kernel (which
    # also writes the rows -D and LSE log2(e)), then its dK/dV kernel
    names = ["attn_fwd", "attn_bwd_dq", "attn_bwd_dkdv"]
    marks = [[T.Event() for _ in range(len(names) + 1)] for _ in range(steps)]
    start, stop = T.Event(), T.Event()
    T.lib().sync()
    start.record()
    for s in range(steps):
        marks[s][0].record()
        T.set_launch_events(marks[s][1:])
        step()
    stop.record()
    T.lib().sync()
    T.set_launch_events([])
    total_ms = T.Event.elapsed(start, stop)
    per = {n: 0.0 for n in names}
    for s in range(steps):
        for i, n in enumerate(names):
            per[n] += T.Event.elapsed(marks[s][i], marks[s][i + 1])
    per = {n: t / steps for n, t in per.items()}
    return total_ms / steps, per


def run_pcie(T, reps=3):
    """The c5 step as a reference user runs it, host to host: fp32 numpy Q, K, V
    and dO (the reference's TinyTensor-from-numpy inputs) uploaded to bf16 device
    buffers (converted in the staging pass), forward + backward, and O, dQ, dK,
    dV downloaded to fp32 numpy.  Reported beside the bench line, never as its
    value (which times the step on HBM-resident inputs)."""
    import numpy as np

    B, H, L, d = C5["B"], C5["H"], C5["L"], C5["d"]
    scale = float(np.float32(1.0 / math.sqrt(d)))
    shp = (B, H, L, d)
    n = B * H * L * d
    rng = np.random.default_rng(5)
    host_in = [rng.standard_normal(shp, dtype=np.float32) for _ in range(4)]
    host_out = [np.empty(shp, np.float32) for _ in range(4)]
    q, k, v, do = (T.DeviceBuffer(shp, "bf16") for _ in range(4))
    o, dq, dk, dv = (T.DeviceBuffer(shp, "bf16") for _ in range(4))
    lse = T.DeviceBuffer((B, H, L), "f32")
    Lb = T.lib()

    def once():
        t0 = time.perf_counter()
        for h, b in zip(host_in, (q, k, v, do)):
            Lb.call("tt_upload_bf16_from_f32", b.ptr, h.ctypes.data, n)
        Lb.sync()
        t1 = time.perf_counter()
        T.attn_fwd(q, k, v, o, lse, scale, True)
        T.attn_bwd(q, k, v, o, lse, do, dq, dk, dv, scale, True)
        Lb.sync()
        t2 = time.perf_counter()
        for h, b in zip(host_out, (o, dq, dk, dv)):
            Lb.call("tt_download_bf16_to_f32", h.ctypes.data, b.ptr, n)
        Lb.sync()
        t3 = time.perf_counter()
        return t3 - t0, t1 - t0, t2 - t1, t3 - t2

    once()
    best = min((once() for _ in range(reps)), key=lambda r: r[0])
    flops = fwdbwd_flops(**C5)
    return {"metric": "c5 fwd+bwd host to host (fp32 numpy in and out, bf16 on the device)",
            "ms_per_step": best[0] * 1e3, "value": flops / best[0] / 1e12, "unit": "TFLOP/s",
            "upload_ms": best[1] * 1e3, "compute_ms": best[2] * 1e3, "download_ms": best[3] * 1e3,
            "host_bytes_per_step": 8 * n * 4, "reps": reps,
            "config": {"workload": "causal attention fwd+bwd, B=4 H=32 L=4096 d=128, fp32 host arrays"}}


def run_decode(T, steps, warmup):
    B, H, Lkv, d = C4["B"], C4["H"], C4["Lkv"], C4["d"]
    scale = float(__import__("numpy").float32(1.0 / math.sqrt(d)))
    q = T.DeviceBuffer((B, H, 1, d), "bf16")
    k = T.DeviceBuffer((B, H, Lkv, d), "bf16")
    v = T.DeviceBuffer((B, H, Lkv, d), "bf16")
    q.fill_normal(4000)
    k.fill_normal(4001)
    v.fill_normal(4002)
    o = T.DeviceBuffer((B, H, 1, d), "bf16")
    lse = T.DeviceBuffer((B, H), "f32")
    prewarm(T, lambda: T.attn_decode(q, k, v, o, lse, scale))
    for _ in range(warmup):
        T.attn_decode(q, k, v, o, lse, scale)
    T.lib().sync()
    # one launch per step when a split covers a whole head (c4), else the split
    # kernel and the combine kernel
    names = ["attn_decode_split", "attn_decode_combine"]
    marks = [[T.Event() for _ in range(3)] for _ in range(steps)]
    start, stop = T.Event(), T.Event()
    start.record()
    for s in range(steps):
        marks[s][0].record()
        T.set_launch_events(marks[s][1:])
        T.attn_decode(q, k, v, o, lse, scale)
        launches = T.launch_events_recorded()
    stop.record()
    T.lib().sync()
    T.set_launch_events([])
    total_ms = T.Event.elapsed(start, stop)
    names = names[:launches]
    per = {n: sum(T.Event.elapsed(marks[s][i], marks[s][i + 1]) for s in range(steps)) / steps
           for i, n in enumerate(names)}
    # The read rate this hardware gives a plain streaming kernel over the same
    # K and V buffers (tt_read_probe: 16-byte loads, 256 KiB per workgroup).
    L = T.lib()
    sink = T.DeviceBuffer((1,), "f32")
    for _ in range(warmup):
        L.call("tt_read_probe", k.ptr, k.nbytes, sink.ptr, None)
        L.call("tt_read_probe", v.ptr, v.nbytes, sink.ptr, None)
    L.sync()
    start.record()
    for _ in range(steps):
        L.call("tt_read_probe", k.ptr, k.nbytes, sink.ptr, None)
        L.call("tt_read_probe", v.ptr, v.nbytes, sink.ptr, None)
    stop.record()
    L.sync()
    probe_ms = T.Event.elapsed(start, stop) / steps
    read_ceiling = {"value": (k.nbytes + v.nbytes) / (probe_ms * 1e-3) / 1e9, "unit": "GB/s",
                    "ms": probe_ms, "bytes": k.nbytes + v.nbytes,
                    "kernel": "k_read_probe (tt_read_probe over the K and V buffers)"}
    del k, v
    return total_ms / steps, per, read_ceiling


# The other BASELINE.json configurations (parity configs c1-c3), each timed
# as one step = forward (+ backward when the config has one) with HIP events
# over `steps` steps, inputs resident in HBM.  fp32 configs are priced
# against the fp32 MFMA peak, bf16 against the bf16 one.
PEAK_FP32_MFMA_TFLOPS = 157.3


class GpuConfig:
    """Shape of a BASELINE.json configuration as the GPU legs time it."""

    def __init__(self, cid, B, H, Lq, Lk, d, dtype, causal, backward, qkv_scale=1.0):
        self.cid, self.B, self.H, self.Lq, self.Lk, self.d = cid, B, H, Lq, Lk, d
        self.dtype, self.causal, self.backward, self.qkv_scale = dtype, causal, backward, qkv_scale
        self.scale = float(__import__("numpy").float32(1.0 / math.sqrt(d)))


GPU_CONFIGS = {
    1: GpuConfig(1, 1, 1, 64, 64, 32, "f32", False, False),
    2: GpuConfig(2, 8, 8, 256, 256, 64, "f32", False, True),
    3: GpuConfig(3, 16, 16, 1024, 1024, 64, "bf16", True, True, 0.5),
    5: GpuConfig(5, C5["B"], C5["H"], C5["L"], C5["L"], C5["d"], "bf16", True, True),
}
# Supported shapes outside BASELINE.json's configurations, timed beside them
# (not graded): fp32 at the largest head dim, causal and not.
EXTRA_CONFIGS = {
    "f32_d128_causal": GpuConfig(0, 2, 16, 2048, 2048, 128, "f32", True, True),
    "f32_d128": GpuConfig(0, 2, 16, 2048, 2048, 128, "f32", False, True),
}


def config_flops(cfg):
    f = (12.0 if cfg.backward else 4.0) * cfg.B * cfg.H * cfg.Lq * cfg.Lk * cfg.d
    return f / 2 if cfg.causal else f


def config_buffers(T, cfg):
    """Device inputs (seeded on the device), output and gradient buffers of `cfg`."""
    dt = cfg.dtype
    qs, ks = (cfg.B, cfg.H, cfg.Lq, cfg.d), (cfg.B, cfg.H, cfg.Lk, cfg.d)
    q, do_ = T.DeviceBuffer(qs, dt), T.DeviceBuffer(qs, dt)
    k, v = T.DeviceBuffer(ks, dt), T.DeviceBuffer(ks, dt)
    for i, b in enumerate((q, k, v, do_)):
        b.fill_normal(6100 + 10 * cfg.cid + i, cfg.qkv_scale if i < 3 else 1.0)
    o = T.DeviceBuffer(qs, dt)
    lse = T.DeviceBuffer(qs[:3], "f32")
    g = [T.DeviceBuffer(qs, dt), T.DeviceBuffer(ks, dt), T.DeviceBuffer(ks, dt)]
    return q, k, v, do_, o, lse, g


def config_step(T, cfg, bufs, part="all"):
    """One step of `cfg`: forward (+ backward); part "fwd" / "bwd" runs one half."""
    q, k, v, do_, o, lse, g = bufs

    def step():
        if part in ("all", "fwd"):
            T.attn_fwd(q, k, v, o, lse, cfg.scale, cfg.causal)
        if cfg.backward and part in ("all", "bwd"):
            T.attn_bwd(q, k, v, o, lse, do_, *g, cfg.scale, cfg.causal)

    return step


def run_config(T, cfg, steps, warmup, part="all"):
    step = config_step(T, cfg, config_buffers(T, cfg), part)
    prewarm(T, step)
    for _ in range(warmup):
        step()
    T.lib().sync()
    a, b = T.Event(), T.Event()
    a.record()
    for _ in range(steps):
        step()
    b.record()
    T.lib().sync()
    return T.Event.elapsed(a, b) / steps


def run_sustain(T, cfg, part, seconds, batch=200):
    """The step of `cfg` (part "all", "fwd" or "bwd") in batches of `batch`
    steps for `seconds`, each batch timed with HIP events: how the rate
    settles while the board runs at its power limit (sample the board's power
    and clock with amd-smi meanwhile)."""
    bufs = config_buffers(T, cfg)
    if part == "bwd":
        config_step(T, cfg, bufs, "fwd")()  # O and LSE for the backward
    step = config_step(T, cfg, bufs, part)
    for _ in range(5):
        step()
    T.lib().sync()
    ms = []
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        a, b = T.Event(), T.Event()
        a.record()
        for _ in range(batch):
            step()
        b.record()
        T.lib().sync()
        ms.append(T.Event.elapsed(a, b) / batch)
    return {"batches": len(ms), "batch_steps": batch, "ms_first_batch": ms[0], "ms_last_batch": ms[-1],
            "ms_median_batch": sorted(ms)[len(ms) // 2], "ms_min_batch": min(ms)}


def config_cpu_baseline(cfg, max_heads, reps=3):
    """The reference's op chain (oracle composition_*_f32, float32 numpy, full
    L x L materialised) on up to `max_heads` heads of the config; returns the
    rate in TFLOP/s of the same algorithmic FLOP count."""
    import numpy as np

    sys.path.insert(0, ROOT)
    from oracle import attn_oracle as orc

    x = orc.seeded_inputs(orc.CONFIGS[cfg.cid])
    heads = [(b, h) for b in range(cfg.B) for h in range(cfg.H)][:max_heads]

    def once():
        for b, h in heads:
            if cfg.backward:
                orc.composition_bwd_f32(x["q"][b, h], x["k"][b, h], x["v"][b, h], x["do"][b, h], cfg.scale, cfg.causal)
            else:
                orc.composition_fwd_f32(x["q"][b, h], x["k"][b, h], x["v"][b, h], cfg.scale, cfg.causal)

    once()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        once()
        ts.append(time.perf_counter() - t0)
    t = sorted(ts)[len(ts) // 2]
    frac = len(heads) / (cfg.B * cfg.H)
    return {"value": config_flops(cfg) * frac / t / 1e12, "unit": "TFLOP/s", "cores": int(_blas_threads()),
            "kind": "port", "seconds": t,
            "sample": f"{len(heads)} of {cfg.B * cfg.H} heads, reference op order in float32 numpy "
                      f"(median of {reps}: {t * 1e3:.1f} ms)"}


def decode_cpu_baseline(heads=256, reps=3):
    """The reference's op chain for one query (Q @ K^T, * s, softmax, @ V) in
    float32 numpy over `heads` (b, h) heads of the decode workload: K/V bytes
    read per second (bf16-sized, as on the GPU)."""
    import numpy as np

    B, H, Lkv, d = C4["B"], C4["H"], C4["Lkv"], C4["d"]
    rng = np.random.default_rng(4)
    k = rng.standard_normal((heads, Lkv, d), dtype=np.float32)
    v = rng.standard_normal((heads, Lkv, d), dtype=np.float32)
    q = rng.standard_normal((heads, 1, d), dtype=np.float32)
    s = np.float32(1.0 / math.sqrt(d))

    def once():
        sc = np.matmul(q, np.swapaxes(k, -1, -2)) * s
        sc = sc - sc.max(axis=-1, keepdims=True)
        e = np.exp(sc)
        return np.matmul(e / e.sum(axis=-1, keepdims=True), v)

    once()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        once()
        ts.append(time.perf_counter() - t0)
    t = sorted(ts)[len(ts) // 2]
    nbytes = heads * (2 * Lkv * d * 2 + 2 * d * 2)
    return {"value": nbytes / t / 1e9, "unit": "GB/s", "cores": int(_blas_threads()), "kind": "port",
            "sample": f"{heads} of {B * H} heads (Lkv={Lkv}, d={d}), float32 numpy, bytes counted as bf16 "
                      f"(median of {reps}: {t * 1e3:.1f} ms)"}


def run_copy(T, steps, warmup, nbytes=1 << 30):
    """Plain fp32 copy (c = 1.0 * a) of `nbytes`: reads and writes exactly
    nbytes each, used to calibrate the profiler's FETCH_SIZE / WRITE_SIZE."""
    n = nbytes // 4
    a = T.DeviceBuffer((n,), "f32")
    c = T.DeviceBuffer((n,), "f32")
    a.fill_normal(1)
    L = T.lib()

    def once():
        L.call("tt_elementwise", 4, 0, c.ptr, a.ptr, None, n, 1.0, 0.0, 0, None)  # TT_EW_SCALE, TT_F32

    prewarm(T, once)
    for _ in range(warmup):
        once()
    start, stop = T.Event(), T.Event()
    L.sync()
    start.record()
    for _ in range(steps):
        once()
    stop.record()
    L.sync()
    ms = T.Event.elapsed(start, stop) / steps
    return ms, 2 * nbytes / (ms * 1e-3) / 1e9


# Row softmax (myLayer.SoftmaxForward / tt_softmax_rows_f32): HBM-bound,
# algorithmic bytes = rows * cols * 4 read + the same written.
SOFTMAX_CASES = [
    dict(name="rows 262144 x 1024 (one wave per row)", rows=262144, cols=1024),
    dict(name="rows 4096 x 65536 (8 workgroups per row, partials exchanged)", rows=4096, cols=65536),
    dict(name="rows 1024 x 262144 (16 workgroups per row, partials exchanged)", rows=1024, cols=262144),
]


def run_softmax(T, steps, warmup, rows, cols):
    x = T.DeviceBuffer((rows, cols), "f32")
    y = T.DeviceBuffer((rows, cols), "f32")
    x.fill_normal(5000, 3.0)
    prewarm(T, lambda: T.softmax_rows(x, y))
    for _ in range(warmup):
        T.softmax_rows(x, y)
    T.lib().sync()
    start, stop = T.Event(), T.Event()
    start.record()
    for _ in range(steps):
        T.softmax_rows(x, y)
    stop.record()
    T.lib().sync()
    ms = T.Event.elapsed(start, stop) / steps
    return ms, 2 * rows * cols * 4 / (ms * 1e-3) / 1e9


# GEMM (tt_gemm_f32 / tt_gemm_bf16, the cudaGemm contract): MFMA-bound,
# 2 m n k FLOP per call.
GEMM_CASES = [
    dict(dtype="f32", m=4096, n=4096, k=4096, ta=False, tb=False),
    dict(dtype="bf16", m=8192, n=8192, k=8192, ta=False, tb=False),
    dict(dtype="bf16", m=8192, n=8192, k=8192, ta=True, tb=True),
]


def run_gemm(T, steps, warmup, dtype, m, n, k, ta, tb):
    A = T.DeviceBuffer((k, m) if ta else (m, k), dtype)
    B = T.DeviceBuffer((n, k) if tb else (k, n), dtype)
    Cb = T.DeviceBuffer((m, n), dtype)
    A.fill_normal(6000)
    B.fill_normal(6001)
    prewarm(T, lambda: T.gemm(ta, tb, m, n, k, 1.0, A, B, 0.0, Cb))
    for _ in range(warmup):
        T.gemm(ta, tb, m, n, k, 1.0, A, B, 0.0, Cb)
    T.lib().sync()
    start, stop = T.Event(), T.Event()
    start.record()
    for _ in range(steps):
        T.gemm(ta, tb, m, n, k, 1.0, A, B, 0.0, Cb)
    stop.record()
    T.lib().sync()
    ms = T.Event.elapsed(start, stop) / steps
    return ms, 2.0 * m * n * k / (ms * 1e-3) / 1e12


# Host <-> device transfers (tt_memcpy_h2d / tt_memcpy_d2h and the converting
# bf16 copies): bound by the host link; the ceiling is the DMA rate from
# pinned host memory, measured beside them.
IO_BYTES = 512 << 20


def run_io(T, reps=4):
    import ctypes as C

    import numpy as np

    L = T.lib()
    n = IO_BYTES // 4
    x = np.random.default_rng(0).standard_normal(n, dtype=np.float32)
    out = np.empty_like(x)
    d = T.DeviceBuffer((n,), "f32")
    db = T.DeviceBuffer((n,), "bf16")
    pin = C.c_void_p()
    L.call("tt_host_malloc", C.byref(pin), IO_BYTES)
    try:
        legs = [
            ("h2d f32, pageable numpy source (staged)", lambda: L.call("tt_memcpy_h2d", d.ptr, x.ctypes.data, IO_BYTES)),
            ("d2h f32, pageable numpy destination (staged)",
             lambda: L.call("tt_memcpy_d2h", out.ctypes.data, d.ptr, IO_BYTES)),
            ("h2d fp32 -> bf16 (converted in the staging pass)",
             lambda: L.call("tt_upload_bf16_from_f32", db.ptr, x.ctypes.data, n)),
            ("d2h bf16 -> fp32 (converted in the staging pass)",
             lambda: L.call("tt_download_bf16_to_f32", out.ctypes.data, db.ptr, n)),
            ("h2d f32, pinned source (direct DMA: ceiling)", lambda: L.call("tt_memcpy_h2d", d.ptr, pin.value, IO_BYTES)),
            ("d2h f32, pinned destination (direct DMA: ceiling)",
             lambda: L.call("tt_memcpy_d2h", pin.value, d.ptr, IO_BYTES)),
        ]
        cases = []
        for name, fn in legs:
            fn()
            ts = []
            for _ in range(reps):
                t0 = time.perf_counter()
                fn()
                ts.append(time.perf_counter() - t0)
            t = min(ts)
            cases.append({"workload": name, "ms": t * 1e3, "value": IO_BYTES / t / 1e9,
                          "unit": "GB/s (of fp32 host bytes)"})
    finally:
        L.call("tt_host_free", pin.value)
    return cases


def softmax_cpu_baseline(rows=16384, cols=1024, reps=3):
    """The reference's softmax formula (Softmaxloss.compute, optimizer/operators.py:611-612,
    the order SoftmaxForward follows on the GPU) in float32 numpy on the host."""
    import numpy as np

    sys.path.insert(0, ROOT)
    from oracle import attn_oracle as orc

    x = np.random.default_rng(0).standard_normal((rows, cols)).astype(np.float32) * 3
    orc.softmax_rows_ref_f32(x)
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        orc.softmax_rows_ref_f32(x)
        ts.append(time.perf_counter() - t0)
    t = sorted(ts)[len(ts) // 2]
    return {"value": 2 * rows * cols * 4 / t / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{rows} x {cols} fp32 rows, numpy max / exp / sum / divide (median of {reps}: {t * 1e3:.1f} ms)"}


def run_gemm_ceiling(n=16384, iters=5):
    """Library bf16 GEMM (torch -> hipBLASLt), n^3, on random N(0,1) and on all-ones
    operands: the MFMA rate a tuned GEMM sustains on this box.  The instruction
    stream is the same for both; the gap is the power the data toggles."""
    import torch

    res = {"gemm": f"bf16 {n}x{n}x{n}, torch.matmul (hipBLASLt)", "iters": iters}
    g = torch.Generator(device="cuda").manual_seed(0)
    for kind in ("random", "ones"):
        if kind == "random":
            a = torch.randn(n, n, device="cuda", dtype=torch.bfloat16, generator=g)
            b = torch.randn(n, n, device="cuda", dtype=torch.bfloat16, generator=g)
        else:
            a = torch.ones(n, n, device="cuda", dtype=torch.bfloat16)
            b = torch.ones(n, n, device="cuda", dtype=torch.bfloat16)
        for _ in range(2):
            c = a @ b
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(iters):
            c = a @ b
        e1.record()
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / iters
        res[f"{kind}_tflops"] = 2.0 * n ** 3 / (ms * 1e-3) / 1e12
        del a, b, c
    torch.cuda.empty_cache()
    res["random_frac_of_peak"] = res["random_tflops"] / PEAK_BF16_TFLOPS
    return res


def cpu_baseline(sample_heads):
    """The reference's op chain in float32 numpy on `sample_heads` heads of
    the headline workload (1 warm-up head, not counted)."""
    import numpy as np

    from oracle import attn_oracle as orc

    cores = _blas_threads()
    L, d = C5["L"], C5["d"]
    scale = float(np.float32(1.0 / math.sqrt(d)))
    rng = np.random.default_rng(5)

    def head():
        return [orc.bf16_round(rng.standard_normal((L, d), dtype=np.float32)) for _ in range(4)]

    q, k, v, do = head()
    orc.composition_bwd_f32(q, k, v, do, scale, True)  # warm-up
    t = 0.0
    for _ in range(sample_heads):
        q, k, v, do = head()
        t0 = time.perf_counter()
        orc.composition_bwd_f32(q, k, v, do, scale, True)  # forward (kept) + backward
        t += time.perf_counter() - t0
    flops = sample_heads * fwdbwd_flops(1, 1, L, d)
    return {
        "value": flops / t / 1e12,
        "unit": "TFLOP/s",
        "cores": int(cores),
        "kind": "port",
        "sample": f"{sample_heads} of the {C5['B'] * C5['H']} (b,h) heads of B=4 H=32 L=4096 d=128 causal "
                  f"fwd+bwd, bf16-valued inputs in fp32, reference op order (full L x L materialised); "
                  f"{t:.2f} s",
    }


def _blas_threads():
    try:
        from threadpoolctl import threadpool_info

        return max([i.get("num_threads", 1) for i in threadpool_info() if i.get("user_api") == "blas"] or [1])
    except Exception:
        return os.cpu_count() or 1


def gemm_cpu_baseline(n=2048, reps=3):
    """The reference's CPU matmul (MatMul.compute = np.matmul in float32,
    optimizer/operators.py:416-419) on the host's BLAS threads."""
    import numpy as np

    rng = np.random.default_rng(0)
    a = rng.standard_normal((n, n), dtype=np.float32)
    b = rng.standard_normal((n, n), dtype=np.float32)
    np.matmul(a, b)
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        np.matmul(a, b)
        ts.append(time.perf_counter() - t0)
    t = sorted(ts)[len(ts) // 2]
    return {"value": 2.0 * n ** 3 / t / 1e12, "unit": "TFLOP/s", "cores": int(_blas_threads()), "kind": "port",
            "sample": f"fp32 {n}^3 np.matmul (median of {reps}: {t * 1e3:.1f} ms)"}


def io_cpu_baseline(T, nbytes=16 << 20):
    """The reference's download path: get_data() (a synchronous copy into a
    std::vector, then a Python list) and np.array of that list, as its
    operators do (optimizer/operators.py:482,511)."""
    import numpy as np

    import myTensor as mt

    x = np.random.default_rng(0).standard_normal(nbytes // 4, dtype=np.float32).reshape(1, -1)
    t = mt.Tensor_float(x, "gpu")
    np.array(t.get_data())
    t0 = time.perf_counter()
    np.array(t.get_data())
    dt = time.perf_counter() - t0
    return {"value": nbytes / dt / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{nbytes >> 20} MiB fp32 tensor, np.array(t.get_data()) ({dt * 1e3:.0f} ms)"}


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--only", choices=["all", "fwdbwd", "configs", "decode", "copy", "ceiling", "softmax", "gemm", "io",
                                       "sustain", "seqsweep", "shapes", "pcie"],
                    default="all",
                    help="run one workload only (for profiler runs; 'copy' is the 1 GiB calibration copy, "
                         "'ceiling' the library bf16 GEMM reference, 'sustain' the --sustain loop, 'seqsweep' "
                         "the c5 step at L = 1024 .. 16384 over the same number of tokens, 'shapes' every head "
                         "size, causal and not, in both dtypes, 'pcie' the c5 step host to host)")
    ap.add_argument("--sustain", default="3:all:8", metavar="CID:PART:SECONDS",
                    help="with --only sustain: config (1, 2, 3 or 5), part (all, fwd or bwd) and duration of a "
                         "loop of 200-step batches")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-heads", type=int, default=128)
    args = ap.parse_args(argv)

    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(heads and batch shard across GPUs with no exchange, so N GPUs run N independent shares).",
              file=sys.stderr)
        return 2

    if args.only == "ceiling":
        # before the library is loaded: torch brings its own HIP runtime
        print(json.dumps({"metric": "library bf16 GEMM TFLOP/s (random vs all-ones operands)",
                          **run_gemm_ceiling()}), flush=True)
        return 0

    import tt_capi as T

    if T.lib().device_count() < 1:
        print("bench.py: no HIP device visible", file=sys.stderr)
        return 1

    if args.only == "sustain":
        cid, part, secs = args.sustain.split(":")
        cfg = GPU_CONFIGS[int(cid)]
        if part not in ("all", "fwd", "bwd"):
            ap.error("--sustain part must be all, fwd or bwd")
        print(json.dumps({"metric": "ms per step over a sustained loop", "config": f"c{cid}", "part": part,
                          **run_sustain(T, cfg, part, float(secs))}), flush=True)
        return 0

    if args.only == "seqsweep":
        # the c5 step (causal, bf16, H = 32, d = 128) and the c3 step (H = 16, d = 64) at other sequence
        # lengths, with the tokens per step of each (B * L = 16384) held fixed
        cases = []
        c3 = GPU_CONFIGS[3]
        fams = ((C5["B"], C5["H"], C5["L"], C5["d"], 1.0), (c3.B, c3.H, c3.Lq, c3.d, c3.qkv_scale))
        for fam, (B0, H, L0, d, qs) in enumerate(fams):
            for i, L in enumerate((1024, 2048, 4096, 8192, 16384)):
                cfg = GpuConfig(50 + 10 * fam + i, (B0 * L0) // L, H, L, L, d, "bf16", True, True, qs)
                ms = run_config(T, cfg, args.steps, args.warmup)
                tf = config_flops(cfg) / (ms * 1e-3) / 1e12
                cases.append({"workload": f"causal fwd+bwd bf16 B={cfg.B} H={cfg.H} L={L} d={cfg.d}", "ms": ms,
                              "value": tf, "unit": "TFLOP/s", "frac_of_peak": tf / PEAK_BF16_TFLOPS})
                print(f"seqsweep d={d} L={L}: {ms:.4f} ms, {tf:.1f} TFLOP/s", file=sys.stderr, flush=True)
        print(json.dumps({"metric": "attn fwd+bwd TFLOP/s by sequence length (same tokens per step)",
                          "steps": args.steps, "warmup": args.warmup, "cases": cases}), flush=True)
        return 0

    if args.only == "shapes":
        # every supported head size, causal and not: bf16 at two sequence lengths over 16384 tokens of 32
        # heads per step, fp32 at one over 4096 tokens of 16 heads; forward alone and forward + backward
        grid = [("bf16", 32, 16384, L, d, c) for d in (32, 64, 128) for c in (True, False) for L in (1024, 4096)]
        grid += [("f32", 16, 4096, 2048, d, c) for d in (32, 64, 128) for c in (True, False)]
        cases = []
        for i, (dt, H, tokens, L, d, causal) in enumerate(grid):
            cfg = GpuConfig(80 + i, tokens // L, H, L, L, d, dt, causal, True)
            peak = PEAK_BF16_TFLOPS if dt == "bf16" else PEAK_FP32_MFMA_TFLOPS
            fwd_flop = config_flops(cfg) / 3  # 4 of the 12 B*H*L^2*d units
            ms = run_config(T, cfg, args.steps, args.warmup)
            fms = run_config(T, cfg, args.steps, args.warmup, part="fwd")
            tf, ftf = config_flops(cfg) / (ms * 1e-3) / 1e12, fwd_flop / (fms * 1e-3) / 1e12
            cases.append({"workload": f"{'causal' if causal else 'full'} attention {dt} B={cfg.B} H={H} L={L} d={d}",
                          "dtype": dt, "fwd_ms": fms, "fwd_tflops": ftf, "step_ms": ms, "step_tflops": tf,
                          "peak": peak, "step_frac_of_peak": tf / peak})
            print(f"shapes {cases[-1]['workload']}: fwd {fms:.4f} ms {ftf:.1f} TF, fwd+bwd {ms:.4f} ms {tf:.1f} TF",
                  file=sys.stderr, flush=True)
        print(json.dumps({"metric": "attn forward and fwd+bwd TFLOP/s by head size, mask and dtype",
                          "steps": args.steps, "warmup": args.warmup, "cases": cases}), flush=True)
        return 0

    out = {
        "metric": "attn fwd+bwd TFLOP/s (% bf16 MFMA peak); decode KV-read HBM GB/s (% peak)",
        "value": None, "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "prewarm_s": PREWARM_S, "ms_per_step": None, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic (on-device seeded N(0,1), bf16)",
        "config": {"workload": "causal attention fwd+bwd, B=4 H=32 L=4096 d=128, bf16 in / fp32 accumulate",
                   "B": C5["B"], "H": C5["H"], "L": C5["L"], "d": C5["d"], "causal": True,
                   "flop_per_step": fwdbwd_flops(**C5)},
    }

    if args.only == "pcie":
        print(json.dumps(run_pcie(T)), flush=True)
        return 0

    if args.only == "copy":
        ms, gbs = run_copy(T, args.steps, args.warmup)
        print(json.dumps({"metric": "calibration copy GB/s (1 GiB read + 1 GiB write)", "value": gbs,
                          "unit": "GB/s", "ms_per_step": ms, "steps": args.steps}), flush=True)
        return 0

    if args.only in ("all", "fwdbwd"):
        ms, per = run_fwdbwd(T, args.steps, args.warmup)
        flops = fwdbwd_flops(**C5)
        out["ms_per_step"] = ms
        out["value"] = flops / (ms * 1e-3) / 1e12
        out["frac_of_peak"] = out["value"] / PEAK_BF16_TFLOPS
        kf = kernel_flops(**C5)
        kernels = {}
        for n, t in per.items():
            tf = kf[n] / (t * 1e-3) / 1e12 if kf[n] else None
            tb = traffic_bytes(n)
            kernels[n] = {"avg_ms": t, "tflops": tf, "frac": (tf / PEAK_BF16_TFLOPS) if tf else None,
                          # measured HBM bytes per launch over this launch time
                          "hbm_gbs": (tb / (t * 1e-3) / 1e9) if tb else None}
        out["kernels"] = kernels
        dom = max(per, key=per.get)
        ach = kf[dom] / (per[dom] * 1e-3) / 1e12
        out["roofline"] = {"bound": "mfma", "kernel": dom, "achieved": ach, "peak": PEAK_BF16_TFLOPS,
                           "unit": "TFLOP/s", "frac": ach / PEAK_BF16_TFLOPS, "traffic": traffic_bytes(dom),
                           "algorithmic_flop_per_launch": kf[dom]}

    if args.only in ("all", "decode"):
        ms, per, read_ceiling = run_decode(T, args.steps, args.warmup)
        nbytes = decode_bytes(**C4)
        gbs = nbytes / (ms * 1e-3) / 1e9
        split = per["attn_decode_split"]
        split_bytes = nbytes - C4["B"] * C4["H"] * C4["d"] * 2  # o is written by the combine kernel
        sgbs = split_bytes / (split * 1e-3) / 1e9
        out["decode"] = {
            "workload": "decode B=64 H=32 Lkv=8192 d=128 bf16", "value": gbs, "unit": "GB/s",
            "ms_per_step": ms, "frac_of_peak": gbs / PEAK_HBM_GBS, "bytes_per_step": nbytes,
            "kernels": {n: {"avg_ms": t} for n, t in per.items()},
            "roofline": {"bound": "hbm", "kernel": "attn_decode_split", "achieved": sgbs, "peak": PEAK_HBM_GBS,
                         "unit": "GB/s", "frac": sgbs / PEAK_HBM_GBS, "traffic": traffic_bytes("attn_decode_split"),
                         "algorithmic_bytes_per_launch": split_bytes},
            "read_ceiling": read_ceiling,
            "frac_of_read_ceiling": sgbs / read_ceiling["value"],
        }
        if not args.no_cpu_baseline:
            out["decode"]["cpu_baseline"] = decode_cpu_baseline()
        if args.only == "decode":
            out["metric"], out["dtype"] = "attn decode KV-read HBM GB/s", "bf16"
            out["config"] = {"workload": out["decode"]["workload"], **C4}
            out["value"], out["unit"], out["ms_per_step"] = gbs, "GB/s", ms
            out["roofline"] = out["decode"]["roofline"]

    if args.only in ("all", "configs"):
        lines = []
        for cid in (1, 2, 3):
            cfg = GPU_CONFIGS[cid]
            ms = run_config(T, cfg, max(args.steps, 20), args.warmup)
            tf = config_flops(cfg) / (ms * 1e-3) / 1e12
            peak = PEAK_BF16_TFLOPS if cfg.dtype == "bf16" else PEAK_FP32_MFMA_TFLOPS
            work = (f"{'causal ' if cfg.causal else ''}attention {'fwd+bwd' if cfg.backward else 'fwd'} {cfg.dtype}, "
                    f"B={cfg.B} H={cfg.H} L={cfg.Lq} d={cfg.d}")
            line = {"config": f"c{cid}", "workload": work, "dtype": cfg.dtype,
                    "flop_per_step": config_flops(cfg), "ms_per_step": ms, "value": tf, "unit": "TFLOP/s",
                    "peak": peak, "frac_of_peak": tf / peak}
            if not args.no_cpu_baseline:
                line["cpu_baseline"] = config_cpu_baseline(cfg, max_heads={1: 1, 2: 64, 3: 32}[cid])
            lines.append(line)
        out["configs"] = lines
        extra = []
        for name, cfg in EXTRA_CONFIGS.items():
            ms = run_config(T, cfg, max(args.steps, 20), args.warmup)
            tf = config_flops(cfg) / (ms * 1e-3) / 1e12
            extra.append({"config": name, "workload": f"{'causal ' if cfg.causal else ''}attention fwd+bwd f32, "
                                                      f"B={cfg.B} H={cfg.H} L={cfg.Lq} d={cfg.d} (not a BASELINE config)",
                          "dtype": "f32", "flop_per_step": config_flops(cfg), "ms_per_step": ms, "value": tf,
                          "unit": "TFLOP/s", "peak": PEAK_FP32_MFMA_TFLOPS, "frac_of_peak": tf / PEAK_FP32_MFMA_TFLOPS})
        out["extra_configs"] = extra

    if args.only in ("all", "softmax"):
        cases = []
        for c in SOFTMAX_CASES:
            ms, gbs = run_softmax(T, args.steps, args.warmup, c["rows"], c["cols"])
            cases.append({"workload": c["name"], "ms": ms, "value": gbs, "unit": "GB/s",
                          "frac_of_peak": gbs / PEAK_HBM_GBS,
                          "algorithmic_bytes_per_launch": 2 * c["rows"] * c["cols"] * 4})
        out["softmax"] = {"cases": cases,
                          "roofline": {"bound": "hbm", "kernel": "k_softmax_reg<16>", "achieved": cases[0]["value"],
                                       "peak": PEAK_HBM_GBS, "unit": "GB/s",
                                       "frac": cases[0]["value"] / PEAK_HBM_GBS,
                                       "traffic": traffic_bytes("softmax_reg")}}
        if not args.no_cpu_baseline:
            out["softmax"]["cpu_baseline"] = softmax_cpu_baseline()
        if args.only == "softmax":
            out["metric"], out["dtype"] = "row softmax HBM GB/s (read + write)", "f32"
            out["config"] = {"workload": cases[0]["workload"]}
            out["value"], out["unit"], out["ms_per_step"] = cases[0]["value"], "GB/s", cases[0]["ms"]
            out["roofline"] = out["softmax"]["roofline"]

    if args.only in ("all", "gemm"):
        cases = []
        for c in GEMM_CASES:
            ms, tf = run_gemm(T, max(3, args.steps // 4), 2, **c)
            peak = PEAK_BF16_TFLOPS if c["dtype"] == "bf16" else PEAK_FP32_MFMA_TFLOPS
            cases.append({"workload": f"{c['dtype']} {c['m']}x{c['n']}x{c['k']} ta={int(c['ta'])} tb={int(c['tb'])}",
                          "ms": ms, "value": tf, "unit": "TFLOP/s", "frac_of_peak": tf / peak, "peak": peak})
        bf = cases[1]
        out["gemm"] = {"cases": cases,
                       "roofline": {"bound": "mfma", "kernel": "k_gemm_dma " + bf["workload"],
                                    "achieved": bf["value"], "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                                    "frac": bf["value"] / PEAK_BF16_TFLOPS,
                                    "traffic": MEASURED_TRAFFIC_MIB["gemm_bf16_nn"] * 2 ** 20}}
        if not args.no_cpu_baseline:
            out["gemm"]["cpu_baseline"] = gemm_cpu_baseline()
        if args.only == "gemm":
            out["metric"], out["dtype"] = "GEMM TFLOP/s (2 m n k per call)", "bf16"
            out["config"] = {"workload": cases[1]["workload"]}
            out["value"], out["unit"], out["ms_per_step"] = cases[1]["value"], "TFLOP/s", cases[1]["ms"]
            out["roofline"] = out["gemm"]["roofline"]

    if args.only in ("all", "io"):
        cases = run_io(T)
        ceil = {"h2d": cases[4]["value"], "d2h": cases[5]["value"]}
        for c in cases[:4]:
            c["frac_of_pinned_dma"] = c["value"] / ceil["h2d" if c["workload"].startswith("h2d") else "d2h"]
        out["io"] = {"bytes": IO_BYTES, "cases": cases}
        if not args.no_cpu_baseline:
            out["io"]["cpu_baseline"] = io_cpu_baseline(T)
        if args.only == "io":
            out["metric"], out["dtype"] = "host -> device staged copy GB/s", "f32"
            out["config"] = {"workload": cases[0]["workload"], "bytes": IO_BYTES}
            out["data"] = "synthetic (host N(0,1) numpy array)"
            out["value"], out["unit"], out["ms_per_step"] = cases[0]["value"], "GB/s", cases[0]["ms"]

    if args.only == "all":
        # context for roofline.frac: what a tuned library GEMM sustains on real data,
        # measured in a child process (torch's HIP runtime is not the library's)
        import subprocess
        r = subprocess.run([sys.executable, os.path.abspath(__file__), "--only", "ceiling"],
                           capture_output=True, text=True, timeout=300)
        try:
            out["mfma_ceiling"] = json.loads(r.stdout.strip().splitlines()[-1])
        except (ValueError, IndexError):
            out["mfma_ceiling"] = {"error": (r.stderr or "no output").strip().splitlines()[-1:]}

    if not args.no_cpu_baseline and args.cpu_heads > 0 and args.only in ("all", "fwdbwd"):
        out["cpu_baseline"] = cpu_baseline(args.cpu_heads)

    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
