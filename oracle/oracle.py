"""CPU oracle for mlx-bun's quantized-inference hot path (ctypes + numpy).

TEST INFRASTRUCTURE ONLY: tests/, ``__graft_entry__.smoke()`` and bench.py's
``cpu_baseline`` leg use this module as the checker.  The product (libmlxq +
the ``mlxq`` host package) never imports it.

The arithmetic is restated in ``oracle.c`` (built into ``oracle/_build``);
this module wraps it and adds the host-side restatements that are pure
bookkeeping: the quantized KV caches' ring mechanics and the batched ring
mask.  Each function names the reference code it follows.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("ORACLE_LIB", os.path.join(HERE, "_build", "liboracle.so"))

F16, F32, BF16 = 9, 10, 12
DTYPES = {"float16": F16, "float32": F32, "bfloat16": BF16}

_lib = None


def build() -> None:
    """Compile oracle.c (gcc) into oracle/_build/liboracle.so."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


def _declare(L: ctypes.CDLL) -> None:
    P = ctypes.c_void_p
    i64, i32, f32 = ctypes.c_int64, ctypes.c_int, ctypes.c_float
    L.oracle_to_t.argtypes = [P, i64, i32, P]
    L.oracle_from_t.argtypes = [P, i64, i32, P]
    L.oracle_quantize.argtypes = [P, i64, i64, i32, i32, i32, P, P, P]
    L.oracle_dequantize.argtypes = [P, P, P, i32, i64, i64, i32, i32, P]
    L.oracle_qmm.argtypes = [P, i64, i64, i64, P, P, P, i32, i64, i64, i32, i32, i32, P]
    sd = [P, i32, i32, i32, i32, i32, i32, P, P, P, P, P, P, i64, i64, P, P, i32, i32, f32, i32, i32]
    L.oracle_sdpa.argtypes = sd + [P]
    L.oracle_sdpa_unfused_t.argtypes = sd + [P]
    L.oracle_sdpa_tiled_t.argtypes = sd + [i32, P]
    for name in ("oracle_quantize", "oracle_dequantize", "oracle_qmm", "oracle_sdpa",
                 "oracle_sdpa_unfused_t", "oracle_sdpa_tiled_t"):
        getattr(L, name).restype = ctypes.c_int


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _t_np(dtype: int):
    return np.float32 if dtype == F32 else np.uint16


# ------------------------------------------------------------------ dtypes

def to_t(x, dtype: int) -> np.ndarray:
    """float -> T bit patterns (uint16 for f16/bf16, float32 for f32), RNE."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=_t_np(dtype))
    lib().oracle_to_t(_p(x), x.size, dtype, _p(out))
    return out


def from_t(t, dtype: int) -> np.ndarray:
    """T bit patterns -> float32."""
    t = np.ascontiguousarray(t, dtype=_t_np(dtype))
    out = np.empty(t.shape, dtype=np.float32)
    lib().oracle_from_t(_p(t), t.size, dtype, _p(out))
    return out


def round_t(x, dtype: int) -> np.ndarray:
    """Round float values to the nearest T value (as float32)."""
    return from_t(to_t(x, dtype), dtype)


# ---------------------------------------------------------------- quantize

def quantize(w, gs: int, bits: int, dtype: int):
    """mx.quantize restatement (oracle.c oracle_quantize).

    w: float array of T values, shape [..., D].  Returns (packed uint32
    [..., D*bits/32], scales T-bits [..., D/gs], biases T-bits [..., D/gs]).
    """
    w = np.ascontiguousarray(w, dtype=np.float32)
    D = w.shape[-1]
    rows = w.size // D if D else 0
    packed = np.empty(w.shape[:-1] + (D * bits // 32,), dtype=np.uint32)
    scales = np.empty(w.shape[:-1] + (D // gs,), dtype=_t_np(dtype))
    biases = np.empty_like(scales)
    rc = lib().oracle_quantize(_p(w), rows, D, gs, bits, dtype, _p(packed), _p(scales), _p(biases))
    if rc:
        raise ValueError(f"oracle_quantize rejected gs={gs} bits={bits} D={D}")
    return packed, scales, biases


def dequantize(packed, scales, biases, gs: int, bits: int, dtype: int) -> np.ndarray:
    """mx.dequantize restatement: T(scale*code + bias) as float32."""
    packed = np.ascontiguousarray(packed, dtype=np.uint32)
    scales = np.ascontiguousarray(scales, dtype=_t_np(dtype))
    biases = np.ascontiguousarray(biases, dtype=_t_np(dtype))
    D = packed.shape[-1] * 32 // bits
    rows = packed.size // packed.shape[-1]
    out = np.empty(packed.shape[:-1] + (D,), dtype=np.float32)
    rc = lib().oracle_dequantize(_p(packed), _p(scales), _p(biases), dtype, rows, D, gs, bits, _p(out))
    if rc:
        raise ValueError("oracle_dequantize rejected its arguments")
    return out


def unpack_codes(packed, bits: int) -> np.ndarray:
    """Integer codes from packed words (little-endian within each uint32)."""
    packed = np.asarray(packed, dtype=np.uint32)
    per = 32 // bits
    shifts = (np.arange(per, dtype=np.uint32) * bits)
    codes = (packed[..., None] >> shifts) & np.uint32((1 << bits) - 1)
    return codes.reshape(packed.shape[:-1] + (packed.shape[-1] * per,))


def qmm(x, w, scales, biases, gs: int, bits: int, dtype: int, transpose: bool = True) -> np.ndarray:
    """quantized_matmul fp32 reference (double accumulation).

    x: [batch, M, K] (or [M, K]); w: [w_batch, N, K*bits/32] (transpose) or
    [w_batch, K, N*bits/32]; returns [batch, M, N] float64.
    """
    x = np.ascontiguousarray(x, dtype=np.float32)
    squeeze = x.ndim == 2
    if squeeze:
        x = x[None]
    w = np.ascontiguousarray(w, dtype=np.uint32)
    if w.ndim == 2:
        w = w[None]
    scales = np.ascontiguousarray(scales, dtype=_t_np(dtype))
    biases = np.ascontiguousarray(biases, dtype=_t_np(dtype))
    batch, M, K = x.shape
    wb = w.shape[0]
    N = w.shape[1] if transpose else w.shape[2] * 32 // bits
    y = np.empty((batch, M, N), dtype=np.float64)
    rc = lib().oracle_qmm(_p(x), batch, M, K, _p(w), _p(scales), _p(biases), dtype, wb, N, gs, bits,
                          int(transpose), _p(y))
    if rc:
        raise ValueError("oracle_qmm rejected its arguments")
    return y[0] if squeeze else y


# -------------------------------------------------------------------- sdpa

def _sdpa_args(q, kq, vq, cap, n_kv, valid_len, ring_off, causal, window, scale, gs, bits, dtype):
    q = np.ascontiguousarray(q, dtype=np.float32)
    B, Hq, Lq, D = q.shape
    kp, ks, kb = (np.ascontiguousarray(a) for a in kq)
    vp, vs, vb = (np.ascontiguousarray(a) for a in vq)
    Hkv = kp.shape[1]
    if cap is None:
        cap = kp.shape[2]
    if n_kv is None:
        n_kv = cap
    vl = None if valid_len is None else np.ascontiguousarray(valid_len, dtype=np.int32)
    ro = None if ring_off is None else np.ascontiguousarray(ring_off, dtype=np.int32)
    keep = (q, kp, ks, kb, vp, vs, vb, vl, ro)
    args = [_p(q), dtype, B, Hq, Hkv, Lq, D, _p(kp), _p(ks), _p(kb), _p(vp), _p(vs), _p(vb),
            cap, n_kv, _p(vl), _p(ro), int(causal), int(window), float(scale), gs, bits]
    return args, keep, (B, Hq, Lq, D)


def sdpa(q, kq, vq, *, scale, gs, bits, dtype, cap=None, n_kv=None, valid_len=None,
         ring_off=None, causal=False, window=0) -> np.ndarray:
    """fp32 reference of quantizedSdpa (double accumulation) -> float64."""
    args, keep, shape = _sdpa_args(q, kq, vq, cap, n_kv, valid_len, ring_off, causal, window,
                                   scale, gs, bits, dtype)
    out = np.empty(shape, dtype=np.float64)
    if lib().oracle_sdpa(*args, _p(out)):
        raise ValueError("oracle_sdpa rejected its arguments")
    del keep
    return out


def sdpa_unfused_t(q, kq, vq, *, scale, gs, bits, dtype, cap=None, n_kv=None, valid_len=None,
                   ring_off=None, causal=False, window=0) -> np.ndarray:
    """quantizedSdpaUnfused with the reference's T rounding points -> float32."""
    args, keep, shape = _sdpa_args(q, kq, vq, cap, n_kv, valid_len, ring_off, causal, window,
                                   scale, gs, bits, dtype)
    out = np.empty(shape, dtype=np.float32)
    if lib().oracle_sdpa_unfused_t(*args, _p(out)):
        raise ValueError("oracle_sdpa_unfused_t rejected its arguments")
    del keep
    return out


def sdpa_tiled_t(q, kq, vq, *, scale, gs, bits, dtype, cap=None, n_kv=None, valid_len=None,
                 ring_off=None, causal=False, window=0, n_chunk=512) -> np.ndarray:
    """quantizedSdpaTiled (512-key chunks, T-typed running state) -> float32."""
    args, keep, shape = _sdpa_args(q, kq, vq, cap, n_kv, valid_len, ring_off, causal, window,
                                   scale, gs, bits, dtype)
    out = np.empty(shape, dtype=np.float32)
    if lib().oracle_sdpa_tiled_t(*args, n_chunk, _p(out)):
        raise ValueError("oracle_sdpa_tiled_t rejected its arguments")
    del keep
    return out


# most negative finite value of each score dtype (mlx finfo(T).min)
FINFO_MIN = {BF16: -3.3895313892515355e38, F16: -65504.0, F32: -3.4028234663852886e38}


def sdpa_array_mask(q, kq, vq, mask, *, scale, gs, bits, dtype, cap=None, n_kv=None, valid_len=None,
                    ring_off=None) -> np.ndarray:
    """quantizedSdpaUnfused under an "array" mask (src/model/gemma4-base.ts:
    1320-1334: where(mask, scores, FINFO_MIN[T]), softmax over the keys), in
    float64 -> [B, Hq, Lq, D].  mask: bool, broadcastable to [B, Lq, n] over
    logical keys j (temporal order); row b's keys are j < valid (valid_len[b]
    capped at cap, else n_kv), key j at slot (ring_off[b] - valid + j) mod cap
    on a ring, else slot j.  q is scaled as T(q * T(scale)) unless scale == 1;
    K and V are dequantized exactly (s * c + b in float64).  A query with every
    key masked gets equal weights on all of them, as the reference's softmax
    over all-FINFO_MIN scores does."""
    q = np.asarray(q, dtype=np.float32)
    B, Hq, Lq, D = q.shape
    kp, ks, kb = kq
    vp, vs, vb = vq
    Hkv = kp.shape[1]
    cap = kp.shape[2] if cap is None else cap
    n_kv = cap if n_kv is None else n_kv

    def deq(p, s_, b_):
        c = unpack_codes(p, bits).astype(np.float64)
        return from_t(s_, dtype).astype(np.float64).repeat(gs, -1) * c + \
            from_t(b_, dtype).astype(np.float64).repeat(gs, -1)

    K, V = deq(kp, ks, kb), deq(vp, vs, vb)  # [B, Hkv, cap, D]
    qs = q.astype(np.float64) if scale == 1.0 else \
        round_t(q * round_t(np.float32(scale), dtype), dtype).astype(np.float64)
    m = np.broadcast_to(np.asarray(mask, dtype=bool).reshape((-1,) + np.shape(mask)[-2:]), (B, Lq, np.shape(mask)[-1]))
    out = np.zeros((B, Hq, Lq, D), dtype=np.float64)
    rep = Hq // Hkv
    for b in range(B):
        valid = n_kv if valid_len is None else min(int(valid_len[b]), cap)
        if valid == 0:
            continue
        j = np.arange(valid)
        slots = (int(ring_off[b]) - valid + j) % cap if ring_off is not None else j
        for h in range(Hq):
            Kb, Vb = K[b, h // rep, slots], V[b, h // rep, slots]
            S = qs[b, h] @ Kb.T  # [Lq, valid]
            S = np.where(m[b, :, :valid], S, FINFO_MIN[dtype])
            S = S - S.max(-1, keepdims=True)
            P = np.exp(S)
            out[b, h] = (P / P.sum(-1, keepdims=True)) @ Vb
    return out


# ----------------------------------------------------------- ring geometry

def ring_slot_mask(valid: int, ring_off: int, cap: int) -> np.ndarray:
    """Physical slots a ring row attends: the `valid` slots written most
    recently before write index `ring_off` (oracle.c row_slot).  Restates the
    per-row window of buildBatchedRotatingMask
    (src/model/batched-rotating.ts:40-75) for decode (N=1)."""
    m = np.zeros(cap, dtype=bool)
    v = min(valid, cap)
    for j in range(v):
        m[(ring_off - v + j) % cap] = True
    return m


def lcg_floats(n: int, seed: int, divisor: float = 2 ** 32) -> np.ndarray:
    """The reference tests' deterministic LCG, (s / divisor) * 2 - 1 per
    step: divisor 2^32 gives [-1, 1) as tests/fused-sdpa.test.ts:29-38;
    randBf16 of tests/fused-decode-kernel.test.ts:16-28 divides by
    0xffffffff (and halves the result)."""
    out = np.empty(n, dtype=np.float32)
    s = seed & 0xFFFFFFFF
    for i in range(n):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        out[i] = np.float32((s / divisor) * 2 - 1)
    return out


def rand_bf16_ref(shape, seed: int) -> np.ndarray:
    """randBf16 of tests/fused-decode-kernel.test.ts:16-28: the LCG over
    0xffffffff, times 0.5, rounded to bf16 (as float32)."""
    n = int(np.prod(shape))
    return round_t((lcg_floats(n, seed, 0xFFFFFFFF) * np.float32(0.5)).reshape(shape), BF16)
