"""Benchmark of the quantized-KV decode attention hot path on one MI355X.

Default (N=1): 4-bit-KV decode attention at 32k context -- B=1, Hq=32,
Hkv=8, D=128, KV length 32768, K/V bf16 ~ N(0,1) quantized 4-bit group 64
on the device, q bf16 ~ N(0,1), scale 1/sqrt(128).  A step is one
quantizedSdpa call over one layer's cache.  Ten distinct cache copies
(10 x 37.8 MB > the 256 MB Infinity Cache) are cycled so each step streams
its cache from HBM.  Steps are captured into one HIP graph so launches run
back to back; value = algorithmic bytes per step / time per step.

Also reported: the 4-bit qmv (x [1, 4096] bf16, W [14336, 4096] 4-bit
group 64) in GB/s, the per-launch kernel time of both (events around single
launches), and the CPU oracle timed on the host on a bounded sample.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "mlx-bun_amd"))

HBM_PEAK_GBS = 8000.0
METRIC = ("qKV SDPA decode GB/s (% of HBM peak) + µs/layer at 4-bit KV, 32k ctx; qmv GB/s")
NSETS = 10
BF16 = 12


def log(msg):
    print(msg, file=sys.stderr, flush=True)


class Timer:
    """HIP events on the library's default stream (the stream every op here
    is issued on)."""

    def __init__(self, lib):
        self.L = lib

    def event(self):
        e = ctypes.c_void_p()
        self.call("mlxq_event_create", ctypes.byref(e))
        return e.value

    def call(self, name, *a):
        from mlxq import _lib

        _lib.call(name, *a)

    def elapsed(self, a, b):
        ms = ctypes.c_float()
        self.call("mlxq_event_elapsed_ms", a, b, ctypes.byref(ms))
        return ms.value

    def per_launch_us(self, fn, n):
        """Mean duration of single launches, each bracketed by its own events."""
        evs = [(self.event(), self.event()) for _ in range(n)]
        for i, (a, b) in enumerate(evs):
            self.call("mlxq_event_record", a, None)
            fn(i)
            self.call("mlxq_event_record", b, None)
        self.call("mlxq_synchronize", None)
        ts = [self.elapsed(a, b) * 1e3 for a, b in evs]
        for a, b in evs:
            self.call("mlxq_event_destroy", a)
            self.call("mlxq_event_destroy", b)
        return float(np.mean(ts)), float(np.median(ts))

    def graph_step_ms(self, fn, steps, warmup):
        """Capture `steps` calls into one graph; warm up, then time one replay."""
        for i in range(warmup):
            fn(i)
        self.call("mlxq_synchronize", None)
        self.call("mlxq_graph_begin", None)
        for i in range(steps):
            fn(i)
        g = ctypes.c_void_p()
        self.call("mlxq_graph_end", None, ctypes.byref(g))
        self.call("mlxq_graph_launch", g, None)  # untimed replay (first-launch costs)
        self.call("mlxq_synchronize", None)
        a, b = self.event(), self.event()
        self.call("mlxq_synchronize", None)
        self.call("mlxq_event_record", a, None)
        self.call("mlxq_graph_launch", g, None)
        self.call("mlxq_event_record", b, None)
        self.call("mlxq_synchronize", None)
        ms = self.elapsed(a, b)
        self.call("mlxq_graph_destroy", g)
        return ms / steps


def rand_bf16(shape, seed):
    from mlxq.array import DeviceArray

    r = np.random.default_rng(seed)
    return DeviceArray.fromFloat32(r.standard_normal(shape, dtype=np.float32), shape, BF16)


# ------------------------------------------------------------------ decode

def decode_workload(B=1, Hq=32, Hkv=8, D=128, N=32768, gs=64, bits=4, seed=0, nsets=NSETS):
    from mlxq import _lib, ops
    from mlxq.array import DeviceArray, Dtype

    k = rand_bf16((B, Hkv, N, D), seed + 1)
    v = rand_bf16((B, Hkv, N, D), seed + 2)
    kq, vq = ops.quantize(k, gs, bits), ops.quantize(v, gs, bits)
    k.dispose()
    v.dispose()
    sets = [(kq, vq)]
    for _ in range(nsets - 1):
        copy = []
        for t in (kq, vq):
            parts = []
            for a in (t.packed, t.scales, t.biases):
                c = DeviceArray.empty(a.shape, a.dtype)
                _lib.call("mlxq_memcpy_dtod", c.ptr, a.ptr, a.nbytes, None)
                parts.append(c)
            copy.append(ops.QuantizedTensor(*parts))
        sets.append(tuple(copy))
    qs = [rand_bf16((B, Hq, 1, D), seed + 10 + i) for i in range(nsets)]
    out = DeviceArray.empty((B, Hq, 1, D), BF16)
    L = _lib.lib()
    scale = ctypes.c_float(D ** -0.5)

    def launch(i):
        kq_, vq_ = sets[i % nsets]
        q = qs[i % nsets]
        rc = L.mlxq_quantized_sdpa(q.ptr, BF16, B, Hq, Hkv, 1, D, kq_.packed.ptr, kq_.scales.ptr, kq_.biases.ptr,
                                   vq_.packed.ptr, vq_.scales.ptr, vq_.biases.ptr, N, N, None, None, 0, 0, scale,
                                   gs, bits, out.ptr, None)
        if rc:
            raise RuntimeError(L.mlxq_last_error().decode())

    kv_bytes = 2 * (kq.packed.nbytes + kq.scales.nbytes + kq.biases.nbytes)
    algo_bytes = kv_bytes + 2 * B * Hq * D * 2  # + q in + out
    return launch, algo_bytes, (sets, qs, out)


def qmv_workload(M=1, N=14336, K=4096, gs=64, bits=4, seed=0, nsets=NSETS):
    from mlxq import _lib, ops
    from mlxq.array import DeviceArray

    r = np.random.default_rng(seed)
    w = DeviceArray.fromFloat32(r.standard_normal((N, K), dtype=np.float32) * 0.02, (N, K), BF16)
    wq = ops.quantize(w, gs, bits)
    w.dispose()
    sets = [wq]
    for _ in range(nsets - 1):
        parts = []
        for a in (wq.packed, wq.scales, wq.biases):
            c = DeviceArray.empty(a.shape, a.dtype)
            _lib.call("mlxq_memcpy_dtod", c.ptr, a.ptr, a.nbytes, None)
            parts.append(c)
        sets.append(ops.QuantizedTensor(*parts))
    xs = [rand_bf16((M, K), seed + 20 + i) for i in range(nsets)]
    y = DeviceArray.empty((M, N), BF16)
    L = _lib.lib()

    def launch(i):
        t = sets[i % nsets]
        rc = L.mlxq_quantized_matmul(xs[i % nsets].ptr, BF16, 1, M, K, t.packed.ptr, t.scales.ptr, t.biases.ptr, 1,
                                     N, gs, bits, 1, y.ptr, None)
        if rc:
            raise RuntimeError(L.mlxq_last_error().decode())

    algo = wq.packed.nbytes + wq.scales.nbytes + wq.biases.nbytes + M * K * 2 + M * N * 2
    return launch, algo, (sets, xs, y)


# -------------------------------------------------------------- cpu oracle

def cpu_baseline(budget_s=15.0):
    """The oracle's decode attention (OpenMP, fp64 accumulation) on the host
    for the same 32k-context workload, as many calls as fit the budget."""
    sys.path.insert(0, ROOT)
    from oracle import oracle as O

    r = np.random.default_rng(0)
    B, Hq, Hkv, D, N = 1, 32, 8, 128, 32768
    k = O.round_t(r.standard_normal((B, Hkv, N, D), dtype=np.float32), O.BF16)
    v = O.round_t(r.standard_normal((B, Hkv, N, D), dtype=np.float32), O.BF16)
    q = O.round_t(r.standard_normal((B, Hq, 1, D), dtype=np.float32), O.BF16)
    kq, vq = O.quantize(k, 64, 4, O.BF16), O.quantize(v, 64, 4, O.BF16)
    calls, t0 = 0, time.perf_counter()
    while True:
        O.sdpa(q, kq, vq, scale=D ** -0.5, gs=64, bits=4, dtype=O.BF16)
        calls += 1
        if time.perf_counter() - t0 > budget_s or calls >= 20:
            break
    dt = (time.perf_counter() - t0) / calls
    algo = 2 * sum(a.nbytes for a in kq) + 2 * B * Hq * D * 2
    cores = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    return {"value": round(algo / dt / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"{calls} call(s) of the full 32k-context decode on the host "
                      f"({dt * 1e3:.1f} ms/call)"}


# --------------------------------------------------------------------- main

def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; multi-GPU sharding is described in DESIGN.md "
                                   "and not launched", "n_gpus": args.gpus}))
        sys.exit(2)

    import mlxq
    from mlxq import _lib

    mlxq.ensure_init(0)
    timer = Timer(_lib.lib())

    log("bench: building 32k decode workload")
    launch, algo_bytes, keep = decode_workload()
    log("bench: decode graph timing")
    ms_step = timer.graph_step_ms(launch, args.steps, args.warmup)
    mean_us, med_us = timer.per_launch_us(launch, 100)
    value = algo_bytes / (ms_step * 1e-3) / 1e9
    achieved = algo_bytes / (mean_us * 1e-6) / 1e9
    del keep

    log("bench: qmv workload")
    qlaunch, qbytes, qkeep = qmv_workload()
    q_ms = timer.graph_step_ms(qlaunch, args.steps, args.warmup)
    q_mean_us, q_med_us = timer.per_launch_us(qlaunch, 100)
    del qkeep

    cpu = None
    if not args.no_cpu:
        log("bench: cpu baseline")
        cpu = cpu_baseline()

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) K/V/q, quantized on device)",
        "config": {
            "workload": "decode SDPA over 4-bit KV cache, 32k context: B=1 Hq=32 Hkv=8 D=128 N=32768, "
                        "group 64, bf16 q/scales/biases, fp32 accumulation",
            "kv_sets_cycled": NSETS,
            "algorithmic_bytes_per_step": algo_bytes,
        },
        "us_per_layer": round(ms_step * 1e3, 3),
        "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
            "kernel": "sdpa_decode_mfma_kernel",
            "launch_us_mean": round(mean_us, 3),
            "launch_us_median": round(med_us, 3),
        },
        "qmv": {
            "workload": "x [1, 4096] bf16 @ W [14336, 4096]^T, 4-bit group 64",
            "GB/s": round(qbytes / (q_ms * 1e-3) / 1e9, 2),
            "us_per_call": round(q_ms * 1e3, 3),
            "kernel_us_mean": round(q_mean_us, 3),
            "kernel_GB/s": round(qbytes / (q_mean_us * 1e-6) / 1e9, 2),
            "algorithmic_bytes": qbytes,
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
