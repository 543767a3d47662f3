"""Benchmark of the quantized-inference hot path on one MI355X.

Headline (the `value`): decode attention over a 4-bit KV cache at 32k
context -- B=1, Hq=32, Hkv=8, D=128, KV length 32768, K/V bf16 ~ N(0,1)
quantized 4-bit group 64 on the device, q bf16 ~ N(0,1), scale 1/sqrt(128).
A step is one quantizedSdpa call over one layer's cache.  Ten distinct cache
copies (10 x 37.8 MB > the 256 MB Infinity Cache) are cycled so each step
streams its cache from HBM.  Steps are captured into one HIP graph so the
launches run back to back; value = algorithmic bytes per step / time per
step.

Also measured in the same run and reported beside it:
  decode_fp16_8bit_1k   B=1 Hq=16 Hkv=4 D=128 N=1024, fp16, 8-bit (latency-bound)
  decode_batched_ring   B=32 Hq=16 Hkv=8 D=256, window 4096, per-row lengths
                        U[512, 32768] and ring offsets U[0, 4096), 4-bit
  qmv_qmm               x [M, 4096] @ W[14336, 4096]^T and x [M, 14336] @
                        W[4096, 14336]^T, 4-bit group 64, M in {1, 4, 16, 64}
  moe_gather_prefill_sorted  gather_qmm over a 512-token chunk's 4096 rows in
                        expert order (SwitchGLU's sorted call), gate_up shape,
                        beside the per-row gather of the same rows
  moe_gather_decode     gather_qmm of one decode token against top-8 of 128
                        stacked 4-bit experts: gate_up [1408, 2816] and down
                        [2816, 704] (the 26B-A4B expert shapes)
  tied_head_qmv         x [1, 2816] @ W[262144, 2816]^T, 4-bit (the tied head,
                        the largest GEMV)
  prefill_chunk         Lq=2048 new queries over 32768 cached keys (4-bit),
                        Hq=32 Hkv=8 D=128, causal
  gemma4_full_attention the 26B-A4B full-attention shape (Hq=16, Hkv=2,
                        D=512, 4-bit): decode at 32k context and a 512-query
                        causal chunk over 8192 keys
  cpu_baseline          the CPU oracle's decode on the host, bounded sample

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--quick] [--only SECTIONS]
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
MFMA_BF16_PEAK_TFLOPS = 2500.0
METRIC = ("qKV SDPA decode GB/s (% of HBM peak) + µs/layer at 4-bit KV, 32k ctx; qmv GB/s")
NSETS = 10
BF16, F16 = 12, 9
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "decode_32k_traffic.json")


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
        """Mean and median of single calls, each bracketed by its own events."""
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
        """Capture `steps` calls into one graph; warm up, then time one replay
        (events recorded on the stream the calls run on, synchronised on
        both sides)."""
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
        self.call("mlxq_event_destroy", a)
        self.call("mlxq_event_destroy", b)
        return ms / steps


def rand_t(shape, seed, dtype=BF16, scale=1.0):
    from mlxq.array import DeviceArray

    r = np.random.default_rng(seed)
    return DeviceArray.fromFloat32(r.standard_normal(shape, dtype=np.float32) * scale, shape, dtype)


rand_bf16 = rand_t


def copy_triple(t):
    from mlxq import _lib, ops
    from mlxq.array import DeviceArray

    parts = []
    for a in (t.packed, t.scales, t.biases):
        c = DeviceArray.empty(a.shape, a.dtype)
        _lib.call("mlxq_memcpy_dtod", c.ptr, a.ptr, a.nbytes, None)
        parts.append(c)
    return ops.QuantizedTensor(*parts)


def quantized_cache(B, Hkv, N, D, gs, bits, seed, dtype):
    from mlxq import ops

    k = rand_t((B, Hkv, N, D), seed + 1, dtype)
    v = rand_t((B, Hkv, N, D), seed + 2, dtype)
    kq, vq = ops.quantize(k, gs, bits), ops.quantize(v, gs, bits)
    k.dispose()
    v.dispose()
    return kq, vq


def sdpa_launcher(qs, sets, out, B, Hq, Hkv, Lq, D, cap, n_kv, gs, bits, dtype, scale, mask=0, vl=None, ro=None):
    from mlxq import _lib

    L = _lib.lib()
    sc = ctypes.c_float(scale)

    def launch(i):
        kq_, vq_ = sets[i % len(sets)]
        q = qs[i % len(qs)]
        rc = L.mlxq_quantized_sdpa(q.ptr, dtype, B, Hq, Hkv, Lq, D, kq_.packed.ptr, kq_.scales.ptr, kq_.biases.ptr,
                                   vq_.packed.ptr, vq_.scales.ptr, vq_.biases.ptr, cap, n_kv,
                                   vl.ptr if vl is not None else None, ro.ptr if ro is not None else None, mask, 0,
                                   sc, gs, bits, out.ptr, None)
        if rc:
            raise RuntimeError(L.mlxq_last_error().decode())

    return launch


# ------------------------------------------------------------------ decode

def decode_workload(B=1, Hq=32, Hkv=8, D=128, N=32768, gs=64, bits=4, seed=0, nsets=NSETS, dtype=BF16):
    from mlxq.array import DeviceArray

    kq, vq = quantized_cache(B, Hkv, N, D, gs, bits, seed, dtype)
    sets = [(kq, vq)] + [(copy_triple(kq), copy_triple(vq)) for _ in range(nsets - 1)]
    qs = [rand_t((B, Hq, 1, D), seed + 10 + i, dtype) for i in range(nsets)]
    out = DeviceArray.empty((B, Hq, 1, D), dtype)
    launch = sdpa_launcher(qs, sets, out, B, Hq, Hkv, 1, D, N, N, gs, bits, dtype, D ** -0.5)
    kv_bytes = 2 * (kq.packed.nbytes + kq.scales.nbytes + kq.biases.nbytes)
    algo_bytes = kv_bytes + 2 * B * Hq * D * 2  # + q in + out
    return launch, algo_bytes, (sets, qs, out)


def batched_ring_workload(B=32, Hq=16, Hkv=8, D=256, W=4096, gs=64, bits=4, seed=3, nsets=2):
    """Per-row valid lengths U[512, 32768] and ring write offsets U[0, W)."""
    from mlxq.array import DeviceArray

    r = np.random.default_rng(seed)
    lens = r.integers(512, 32769, B).astype(np.int32)
    ring = r.integers(0, W, B).astype(np.int32)
    vl = DeviceArray.fromNumpy(lens, 7)
    ro = DeviceArray.fromNumpy(ring, 7)
    sets = [quantized_cache(B, Hkv, W, D, gs, bits, seed + 20 * i, BF16) for i in range(nsets)]
    qs = [rand_t((B, Hq, 1, D), seed + 50 + i) for i in range(nsets)]
    out = DeviceArray.empty((B, Hq, 1, D), BF16)
    launch = sdpa_launcher(qs, sets, out, B, Hq, Hkv, 1, D, W, W, gs, bits, BF16, 1.0, vl=vl, ro=ro)
    per_token = 2 * Hkv * (D * bits // 8 + 2 * 2 * (D // gs))  # K and V codes + scales + biases
    algo = int(np.minimum(lens, W).sum()) * per_token + 2 * B * Hq * D * 2
    return launch, algo, (sets, qs, out, vl, ro)


# --------------------------------------------------------------------- qmv

def qmv_workload(M=1, N=14336, K=4096, gs=64, bits=4, seed=0, nsets=NSETS):
    from mlxq import _lib, ops
    from mlxq.array import DeviceArray

    w = rand_t((N, K), seed, BF16, 0.02)
    wq = ops.quantize(w, gs, bits)
    w.dispose()
    sets = [wq] + [copy_triple(wq) for _ in range(nsets - 1)]
    xs = [rand_t((M, K), seed + 20 + i) for i in range(nsets)]
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


# ------------------------------------------------------------ MoE gather

def moe_gather_workload(N, K, E=128, topk=8, B=1, gs=64, bits=4, seed=60, nsets=NSETS):
    """SwitchGLU decode over E stacked 4-bit experts [E, N, K]: x [B, 1, K]
    against top-k indices [B, 1, k] (gather_qmm, output element i reading x
    row i // k).  16 experts are quantized and copied into the E slots (E
    distinct buffers, E x expert bytes > the Infinity Cache); each step takes
    the next of nsets seeded top-k selections."""
    from mlxq import _lib, ops
    from mlxq.array import DeviceArray

    src = ops.quantize(rand_t((16, N, K), seed, BF16, 0.02), gs, bits)
    parts = []
    for a in (src.packed, src.scales, src.biases):
        full = DeviceArray.empty((E,) + a.shape[1:], a.dtype)
        per = a.nbytes // 16
        for e in range(E):
            _lib.call("mlxq_memcpy_dtod", full.ptr + e * per, a.ptr + (e % 16) * per, per, None)
        parts.append(full)
    src.dispose()
    wp, ws, wb = parts
    r = np.random.default_rng(seed + 1)
    idx = [DeviceArray.fromNumpy(np.stack([r.choice(E, topk, replace=False) for _ in range(B)]).astype(np.uint32)
                                 .ravel(), 3) for _ in range(nsets)]
    xmap = DeviceArray.fromNumpy(np.arange(B * topk, dtype=np.int32) // topk, 7)
    xs = [rand_t((B, 1, K), seed + 20 + i) for i in range(nsets)]
    y = DeviceArray.empty((B * topk, 1, N), BF16)
    L = _lib.lib()

    def launch(i):
        rc = L.mlxq_gather_qmm(xs[i % nsets].ptr, BF16, B, B * topk, 1, K, xmap.ptr, idx[i % nsets].ptr, wp.ptr,
                               ws.ptr, wb.ptr, E, N, gs, bits, 1, y.ptr, None)
        if rc:
            raise RuntimeError(L.mlxq_last_error().decode())

    expert_bytes = N * K * bits // 8 + 2 * 2 * N * (K // gs)
    algo = B * topk * expert_bytes + B * K * 2 + B * topk * N * 2
    return launch, algo, (parts, idx, xmap, xs, y)


def moe_sorted_workload(N, K, E=128, tokens=512, topk=8, gs=64, bits=4, seed=90):
    """SwitchGLU over a prefill chunk: tokens x topk (row, expert) pairs,
    rows gathered in expert order (x [rows, 1, K], indices sorted), against
    E stacked 4-bit experts [E, N, K] (16 quantized experts copied into the E
    slots).  Returns launchers for the sorted (grouped GEMM) and the per-row
    gather over the same rows, and the algorithmic bytes (each present
    expert once, x in, y out)."""
    from mlxq import _lib, ops
    from mlxq.array import DeviceArray

    src = ops.quantize(rand_t((16, N, K), seed, BF16, 0.02), gs, bits)
    parts = []
    for a in (src.packed, src.scales, src.biases):
        full = DeviceArray.empty((E,) + a.shape[1:], a.dtype)
        per = a.nbytes // 16
        for e in range(E):
            _lib.call("mlxq_memcpy_dtod", full.ptr + e * per, a.ptr + (e % 16) * per, per, None)
        parts.append(full)
    src.dispose()
    wp, ws, wb = parts
    r = np.random.default_rng(seed + 1)
    sel = np.stack([r.choice(E, topk, replace=False) for _ in range(tokens)]).ravel()
    idx_h = np.sort(sel).astype(np.uint32)
    rows = idx_h.size
    idx = DeviceArray.fromNumpy(idx_h, 3)
    x = rand_t((rows, 1, K), seed + 2)
    y = DeviceArray.empty((rows, 1, N), BF16)
    L = _lib.lib()

    def sorted_launch(i):
        rc = L.mlxq_gather_qmm_sorted(x.ptr, BF16, rows, K, idx.ptr, wp.ptr, ws.ptr, wb.ptr, E, N, gs, bits, y.ptr,
                                      None)
        if rc:
            raise RuntimeError(L.mlxq_last_error().decode())

    def per_row_launch(i):
        rc = L.mlxq_gather_qmm(x.ptr, BF16, rows, rows, 1, K, None, idx.ptr, wp.ptr, ws.ptr, wb.ptr, E, N, gs, bits,
                               1, y.ptr, None)
        if rc:
            raise RuntimeError(L.mlxq_last_error().decode())

    expert_bytes = N * K * bits // 8 + 2 * 2 * N * (K // gs)
    algo = len(np.unique(idx_h)) * expert_bytes + rows * K * 2 + rows * N * 2
    flops = 2 * rows * N * K
    return sorted_launch, per_row_launch, algo, flops, (parts, idx, x, y)


# ------------------------------------------------------------- tied head

def tied_head_workload(vocab=262144, H=2816, gs=64, bits=4, seed=80):
    """QuantizedEmbedding.asLinear at the 26B-A4B table size: x [1, H] @
    W[vocab, H]^T, 4-bit (415 MB of table, more than the Infinity Cache, so
    one copy streams from HBM).  A 16384-row block is quantized and copied
    into every slot of the table."""
    from mlxq import _lib, ops
    from mlxq.array import DeviceArray

    blk = 16384
    src = ops.quantize(rand_t((blk, H), seed, BF16, 0.02), gs, bits)
    parts = []
    for a in (src.packed, src.scales, src.biases):
        full = DeviceArray.empty((vocab,) + a.shape[1:], a.dtype)
        for r in range(vocab // blk):
            _lib.call("mlxq_memcpy_dtod", full.ptr + r * a.nbytes, a.ptr, a.nbytes, None)
        parts.append(full)
    src.dispose()
    wp, ws, wb = parts
    xs = [rand_t((1, H), seed + 1 + i) for i in range(2)]
    y = DeviceArray.empty((1, vocab), BF16)
    L = _lib.lib()

    def launch(i):
        rc = L.mlxq_quantized_matmul(xs[i % 2].ptr, BF16, 1, 1, H, wp.ptr, ws.ptr, wb.ptr, 1, vocab, gs, bits, 1,
                                     y.ptr, None)
        if rc:
            raise RuntimeError(L.mlxq_last_error().decode())

    algo = wp.nbytes + ws.nbytes + wb.nbytes + H * 2 + vocab * 2
    return launch, algo, (parts, xs, y)


# ----------------------------------------------------------------- prefill

def prefill_workload(B=1, Hq=32, Hkv=8, D=128, Lq=2048, N=32768, gs=64, bits=4, seed=7):
    from mlxq.array import DeviceArray

    kq, vq = quantized_cache(B, Hkv, N, D, gs, bits, seed, BF16)
    qs = [rand_t((B, Hq, Lq, D), seed + 5)]
    out = DeviceArray.empty((B, Hq, Lq, D), BF16)
    launch = sdpa_launcher(qs, [(kq, vq)], out, B, Hq, Hkv, Lq, D, N, N, gs, bits, BF16, D ** -0.5, mask=1)
    pairs = sum(min(N, N - Lq + i + 1) for i in range(Lq))
    flops = 4 * D * pairs * Hq
    return launch, flops, (kq, vq, qs, out)


# -------------------------------------------------------------- cpu oracle

def cpu_baseline(budget_s=15.0):
    """The oracle's decode attention (C, OpenMP, fp64 accumulation) on the
    host for the same 32k-context workload, as many calls as fit the budget."""
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
            "sample": f"{calls} call(s) of the full 32k-context 4-bit decode (B=1 Hq=32 Hkv=8 D=128) on the "
                      f"host, {dt * 1e3:.1f} ms/call"}


def traffic_bytes():
    """HBM bytes per decode call from the committed rocprofv3 PMC summary
    (FETCH_SIZE + WRITE_SIZE scaled by the copy-kernel calibration), or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            return json.load(f).get("bytes_per_call")
    except (OSError, ValueError):
        return None


# --------------------------------------------------------------------- main

SECTIONS = ("decode", "qmm", "decode_1k", "ring", "moe", "moe_sorted", "tied_head", "prefill", "gemma4")


def copy_calibration(timer, nbytes=256 << 20, steps=20):
    """A device-to-device copy of a known size (the reference point that
    scales rocprofv3's FETCH_SIZE / WRITE_SIZE counters to bytes)."""
    from mlxq import _lib
    from mlxq.array import DeviceArray

    src, dst = DeviceArray.empty((nbytes,), 3), DeviceArray.empty((nbytes,), 3)
    src_p, dst_p = src.ptr, dst.ptr
    ms = timer.graph_step_ms(lambda i: _lib.call("mlxq_memcpy_dtod", dst_p, src_p, nbytes // 4 * 4, None), steps, 2)
    return {"bytes_per_copy": nbytes // 4 * 4, "us_per_copy": round(ms * 1e3, 2),
            "GB/s (read + write)": round(2 * nbytes / (ms * 1e-3) / 1e9, 1)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--quick", action="store_true", help="headline decode and qmv M=1 only")
    ap.add_argument("--only", default=None,
                    help="comma list of sections to run (profiling runs): " + ", ".join(SECTIONS) +
                         ", copy (a 256 MiB device copy: the PMC byte-counter reference)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "runs on one GPU only: decode shards over (batch, kv head) or splits the "
                                   "sequence with one all-gather of fp32 partials, which is not launched here",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    if args.only:
        want = set(args.only.split(","))
        bad = want - set(SECTIONS) - {"copy"}
        if bad:
            ap.error(f"unknown sections {sorted(bad)}")
    else:
        want = {"decode", "qmm"} if args.quick else set(SECTIONS)
    run = want.__contains__

    import mlxq
    from mlxq import _lib

    mlxq.ensure_init(0)
    timer = Timer(_lib.lib())

    value = ms_step = mean_us = med_us = algo_bytes = None
    if run("decode"):
        log("bench: 32k decode (headline)")
        launch, algo_bytes, keep = decode_workload()
        ms_step = timer.graph_step_ms(launch, args.steps, args.warmup)
        mean_us, med_us = timer.per_launch_us(launch, 100)
        value = algo_bytes / (ms_step * 1e-3) / 1e9
        del keep

    extra = {}
    qmm = []
    if run("qmm"):
        log("bench: qmv / qmm")
        shapes = [(1, 14336, 4096)] if args.quick else [(m, n, k) for (n, k) in ((14336, 4096), (4096, 14336))
                                                         for m in (1, 4, 16, 64)]
        for M, N, K in shapes:
            ql, qb, qk = qmv_workload(M=M, N=N, K=K)
            q_ms = timer.graph_step_ms(ql, 200, 20)
            qmm.append({"M": M, "N": N, "K": K, "us_per_call": round(q_ms * 1e3, 3),
                        "GB/s": round(qb / (q_ms * 1e-3) / 1e9, 1),
                        "pct_hbm_peak": round(100 * qb / (q_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 1),
                        "TFLOP/s": round(2 * M * N * K / (q_ms * 1e-3) / 1e12, 2), "algorithmic_bytes": qb})
            del qk
        extra["qmv_qmm"] = qmm

    if run("decode_1k"):
        log("bench: decode fp16 8-bit 1k")
        l1, b1, k1 = decode_workload(B=1, Hq=16, Hkv=4, D=128, N=1024, gs=64, bits=8, dtype=F16)
        ms1 = timer.graph_step_ms(l1, 200, 20)
        extra["decode_fp16_8bit_1k"] = {"us_per_call": round(ms1 * 1e3, 3), "algorithmic_bytes": b1,
                                        "GB/s": round(b1 / (ms1 * 1e-3) / 1e9, 1)}
        del k1
    if run("ring"):
        log("bench: batched ring decode")
        l3, b3, k3 = batched_ring_workload()
        ms3 = timer.graph_step_ms(l3, 200, 20)
        extra["decode_batched_ring"] = {"us_per_call": round(ms3 * 1e3, 3), "algorithmic_bytes": b3,
                                        "GB/s": round(b3 / (ms3 * 1e-3) / 1e9, 1),
                                        "pct_hbm_peak": round(100 * b3 / (ms3 * 1e-3) / 1e9 / HBM_PEAK_GBS, 1)}
        del k3
    if run("moe"):
        log("bench: MoE gather_qmm decode")
        moe = {}
        for name, (n, k) in (("gate_up", (1408, 2816)), ("down", (2816, 704))):
            lm, bm, km = moe_gather_workload(n, k)
            msm = timer.graph_step_ms(lm, 200, 20)
            moe[name] = {"N": n, "K": k, "us_per_call": round(msm * 1e3, 3), "algorithmic_bytes": bm,
                         "GB/s": round(bm / (msm * 1e-3) / 1e9, 1),
                         "pct_hbm_peak": round(100 * bm / (msm * 1e-3) / 1e9 / HBM_PEAK_GBS, 1)}
            del km
        extra["moe_gather_decode"] = moe
    if run("moe_sorted"):
        log("bench: MoE gather_qmm, sorted prefill rows")
        ls_, lr_, bs_, fs_, ks_ = moe_sorted_workload(1408, 2816)
        mss = timer.graph_step_ms(ls_, 50, 5)
        msr = timer.graph_step_ms(lr_, 5, 1)
        extra["moe_gather_prefill_sorted"] = {
            "workload": "gate_up [1408, 2816] 4-bit, 512 tokens x top-8 of 128 experts = 4096 rows in expert order",
            "us_per_call": round(mss * 1e3, 2), "per_row_us_per_call": round(msr * 1e3, 2),
            "algorithmic_bytes": bs_, "GB/s": round(bs_ / (mss * 1e-3) / 1e9, 1),
            "TFLOP/s": round(fs_ / (mss * 1e-3) / 1e12, 1)}
        del ks_
    if run("tied_head"):
        log("bench: tied head")
        lh, bh, kh = tied_head_workload()
        msh = timer.graph_step_ms(lh, 200, 10)
        extra["tied_head_qmv"] = {"workload": "x [1, 2816] @ W[262144, 2816]^T, 4-bit group 64",
                                  "us_per_call": round(msh * 1e3, 2), "algorithmic_bytes": bh,
                                  "GB/s": round(bh / (msh * 1e-3) / 1e9, 1),
                                  "pct_hbm_peak": round(100 * bh / (msh * 1e-3) / 1e9 / HBM_PEAK_GBS, 1)}
        del kh
    if run("prefill"):
        log("bench: chunked prefill")
        l5, f5, k5 = prefill_workload()
        m5, md5 = timer.per_launch_us(l5, 10)
        extra["prefill_chunk"] = {"us_per_call": round(md5, 1), "flops": f5,
                                  "TFLOP/s": round(f5 / (md5 * 1e-6) / 1e12, 1),
                                  "pct_mfma_bf16_peak": round(100 * f5 / (md5 * 1e-6) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 1)}
        del k5
    if run("gemma4"):
        log("bench: gemma4 full attention (D 512)")
        g4 = {}
        lg, bg, kg = decode_workload(B=1, Hq=16, Hkv=2, D=512, N=32768, gs=64, bits=4)
        msg = timer.graph_step_ms(lg, 200, 20)
        g4["decode_32k"] = {"us_per_call": round(msg * 1e3, 2), "algorithmic_bytes": bg,
                            "GB/s": round(bg / (msg * 1e-3) / 1e9, 1),
                            "pct_hbm_peak": round(100 * bg / (msg * 1e-3) / 1e9 / HBM_PEAK_GBS, 1)}
        del kg
        lp, fp, kpw = prefill_workload(Hq=16, Hkv=2, D=512, Lq=512, N=8192)
        mp, mdp = timer.per_launch_us(lp, 5)
        g4["prefill_512x8192"] = {"us_per_call": round(mdp, 1), "flops": fp,
                                  "TFLOP/s": round(fp / (mdp * 1e-6) / 1e12, 1),
                                  "pct_mfma_bf16_peak": round(100 * fp / (mdp * 1e-6) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 1)}
        del kpw
        extra["gemma4_full_attention"] = g4
    if run("copy"):
        log("bench: device copy (counter reference)")
        extra["device_copy"] = copy_calibration(timer)

    cpu = None
    if not args.no_cpu and run("decode"):
        log("bench: cpu baseline")
        cpu = cpu_baseline()

    if value is None:
        # a profiling run without the headline section: report what ran
        print(json.dumps({"metric": METRIC, "value": None, "sections": sorted(want), "other_configs": extra}),
              flush=True)
        return
    qmv1 = qmm[0] if qmm else None
    traffic = traffic_bytes()
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
        "data": "synthetic (seeded N(0,1) K/V/q and N(0, 0.02^2) weights, quantized on the device)",
        "config": {
            "workload": "decode SDPA over a 4-bit KV cache, 32k context: B=1 Hq=32 Hkv=8 D=128 N=32768, "
                        "group 64, bf16 q/scales/biases, fp32 accumulation",
            "kv_sets_cycled": NSETS,
            "algorithmic_bytes_per_step": algo_bytes,
        },
        "us_per_layer": round(ms_step * 1e3, 3),
        "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "roofline": {
            "bound": "hbm",
            "achieved": round(value, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(value / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_source": ("not measured in this run: HBM bytes per decode call (partial + merge kernel) from "
                               "the committed rocprofv3 FETCH_SIZE / WRITE_SIZE passes over this workload, scaled "
                               "by a 256 MiB device copy of the same run (profiles/decode_32k_traffic.json, "
                               "profiles/bench_kernels_pmc_counters.txt)")
            if traffic is not None else None,
            "kernel": "decode call = sdpa_decode_mfma_kernel + sdpa_decode_merge_kernel (graph-replayed, "
                      "per-step time)",
            "single_call_us_mean": round(mean_us, 3),
            "single_call_us_median": round(med_us, 3),
        },
        "qmv": ({"workload": "x [1, 4096] bf16 @ W [14336, 4096]^T, 4-bit group 64",
                 "GB/s": qmv1["GB/s"], "us_per_call": qmv1["us_per_call"], "pct_hbm_peak": qmv1["pct_hbm_peak"]}
                if qmv1 else None),
        "other_configs": extra,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
