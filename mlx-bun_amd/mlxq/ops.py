"""The reference's quantized op surface over libmlxq.

Names, argument meaning and error behaviour follow src/mlx/ops.ts
(quantize :615-641, dequantize :212-225, quantizedMatmul :171-184,
gatherQmm :186-204, quantizedMatmulQT :760-775) and src/model/gemma4-base.ts (Mask :21-32,
quantizedSdpa :1560-1578, createCausalMask :1595-1615).  Every op runs
asynchronously on the library's default stream; reading a result back
(toFloat32/rawNumpy) synchronises.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional

import numpy as np

from . import _lib
from .array import DeviceArray, Dtype, itemsize

_FLOATS = (Dtype.float16, Dtype.bfloat16, Dtype.float32)


@dataclass
class QuantSpec:
    bits: int
    groupSize: int
    mode: str = "affine"


@dataclass
class QuantizedTensor:
    """(packed uint32, scales T, biases T) -- ops.QuantizedTensor."""

    packed: DeviceArray
    scales: DeviceArray
    biases: DeviceArray

    def dispose(self) -> None:
        for a in (self.packed, self.scales, self.biases):
            a.dispose()


def _need_contiguous(a: DeviceArray, what: str) -> None:
    if not a.is_contiguous():
        raise ValueError(f"{what} must be contiguous")


def _check_mode(mode: str) -> None:
    if mode != "affine":
        raise ValueError(f"quantization mode {mode!r} is not supported (affine only)")


def quantize(w: DeviceArray, groupSize: int, bits: int, mode: str = "affine") -> QuantizedTensor:
    """mx.quantize: w [..., D] -> packed [..., D*bits/32] u32, scales/biases [..., D/groupSize]."""
    _check_mode(mode)
    _need_contiguous(w, "quantize input")
    if w.dtype not in _FLOATS:
        raise ValueError("quantize expects a floating-point array")
    D = w.shape[-1]
    rows = w.size // D if D else 0
    lead = w.shape[:-1]
    packed = DeviceArray.empty(lead + (D * bits // 32,), Dtype.uint32)
    scales = DeviceArray.empty(lead + (D // groupSize,), w.dtype)
    biases = DeviceArray.empty(lead + (D // groupSize,), w.dtype)
    _lib.call("mlxq_quantize", w.ptr, w.dtype, rows, D, groupSize, bits, packed.ptr, scales.ptr, biases.ptr, None)
    return QuantizedTensor(packed, scales, biases)


def dequantize(w: DeviceArray, scales: DeviceArray, biases: Optional[DeviceArray], spec: QuantSpec) -> DeviceArray:
    """mx.dequantize: T(scale * code + bias), shape [..., D]."""
    _check_mode(spec.mode)
    if biases is None:
        raise ValueError("affine dequantize requires biases")
    for a, n in ((w, "packed"), (scales, "scales"), (biases, "biases")):
        _need_contiguous(a, n)
    D = w.shape[-1] * 32 // spec.bits
    rows = w.size // w.shape[-1]
    out = DeviceArray.empty(w.shape[:-1] + (D,), scales.dtype)
    _lib.call("mlxq_dequantize", w.ptr, scales.ptr, biases.ptr, scales.dtype, rows, D, spec.groupSize, spec.bits,
              out.ptr, None)
    return out


def quantizedMatmul(x: DeviceArray, w: DeviceArray, scales: DeviceArray, biases: Optional[DeviceArray],
                    spec: QuantSpec, transpose: bool = True) -> DeviceArray:
    """mx.quantized_matmul.  x [..., M, K]; w [..., N, K*bits/32] (transpose)
    or [..., K, N*bits/32]; leading dims of w broadcast over x's (size-1 or
    equal).  Returns [..., M, N] in x's dtype, fp32 accumulation."""
    _check_mode(spec.mode)
    if biases is None:
        raise ValueError("affine quantized_matmul requires biases")
    for a, n in ((x, "x"), (w, "w"), (scales, "scales"), (biases, "biases")):
        _need_contiguous(a, n)
    if x.dtype != scales.dtype:
        raise ValueError("x and scales must share a dtype")
    K = x.shape[-1]
    M = x.shape[-2] if len(x.shape) >= 2 else 1
    x_lead = x.shape[:-2] if len(x.shape) >= 2 else ()
    w_lead = w.shape[:-2]
    batch = int(np.prod(x_lead)) if x_lead else 1
    w_batch = int(np.prod(w_lead)) if w_lead else 1
    if transpose:
        N = w.shape[-2]
        if w.shape[-1] * 32 // spec.bits != K:
            raise ValueError(f"quantized_matmul: x has K={K}, w holds {w.shape[-1] * 32 // spec.bits}")
    else:
        N = w.shape[-1] * 32 // spec.bits
        if w.shape[-2] != K:
            raise ValueError(f"quantized_matmul: x has K={K}, w has {w.shape[-2]} rows")
    out_shape = (x.shape[:-1] + (N,)) if len(x.shape) >= 2 else (N,)
    y = DeviceArray.empty(out_shape, x.dtype)
    _lib.call("mlxq_quantized_matmul", x.ptr, x.dtype, batch, M, K, w.ptr, scales.ptr, biases.ptr, w_batch, N,
              spec.groupSize, spec.bits, int(bool(transpose)), y.ptr, None)
    return y


def quantizedMatmulQT(x: DeviceArray, qt: QuantizedTensor, transpose: bool, groupSize: int,
                      bits: int) -> DeviceArray:
    """quantized_matmul against a QuantizedTensor (x @ qt^T or x @ qt)."""
    return quantizedMatmul(x, qt.packed, qt.scales, qt.biases, QuantSpec(bits, groupSize), transpose)


def gather_batch_maps(x_lead, idx_shape):
    """Broadcast x's leading dims against rhs_indices' shape, as gather_qmm
    broadcasts its batch dims: returns (out_lead, x_map), x_map[i] being the x
    batch element output element i reads, or None when that is i itself."""
    x_lead, idx_shape = tuple(x_lead), tuple(idx_shape)
    out_lead = tuple(np.broadcast_shapes(x_lead, idx_shape))
    if x_lead == out_lead:
        return out_lead, None
    x_batch = int(np.prod(x_lead)) if x_lead else 1
    xm = np.broadcast_to(np.arange(x_batch, dtype=np.int32).reshape(x_lead), out_lead).ravel()
    return out_lead, np.ascontiguousarray(xm)


def gatherQmm(x: DeviceArray, w: DeviceArray, scales: DeviceArray, biases: Optional[DeviceArray],
              rhsIndices: DeviceArray, spec: QuantSpec, sortedIndices: bool, transpose: bool = True) -> DeviceArray:
    """mx.gather_qmm with rhs_indices (src/mlx/ops.ts:186-204), as
    QuantizedSwitchLinear.forward calls it (src/model/gemma4-base.ts:1642).
    x [..., M, K]; w [E, N, K*bits/32] (transpose) or [E, K, N*bits/32];
    rhsIndices (uint32 or int32) selects the expert per output batch element,
    its shape broadcasting with x's leading dims.  Returns
    broadcast(x[..., :-2], rhsIndices) + [M, N] in x's dtype.  sortedIndices
    is MLX's scheduling hint, results do not depend on it: for SwitchGLU's
    sorted call (rows gathered in expert order, x [rows, 1, K], indices
    [rows], src/model/gemma4.ts:441-473) it runs each expert's rows as GEMM
    blocks (mlxq_gather_qmm_sorted) instead of one matrix-vector product a
    row."""
    _check_mode(spec.mode)
    if biases is None:
        raise ValueError("affine gather_qmm requires biases")
    for a, n in ((x, "x"), (w, "w"), (scales, "scales"), (biases, "biases"), (rhsIndices, "rhsIndices")):
        _need_contiguous(a, n)
    if x.dtype != scales.dtype:
        raise ValueError("x and scales must share a dtype")
    if rhsIndices.dtype not in (3, 7):
        raise ValueError("rhsIndices must be uint32 or int32")
    if len(w.shape) != 3:
        raise ValueError("gather_qmm: w must be [experts, rows, packed]")
    if len(x.shape) < 2:
        raise ValueError("gather_qmm: x must be [..., M, K]")
    K, M = x.shape[-1], x.shape[-2]
    E = w.shape[0]
    if transpose:
        N = w.shape[1]
        if w.shape[2] * 32 // spec.bits != K:
            raise ValueError(f"gather_qmm: x has K={K}, w holds {w.shape[2] * 32 // spec.bits}")
    else:
        N = w.shape[2] * 32 // spec.bits
        if w.shape[1] != K:
            raise ValueError(f"gather_qmm: x has K={K}, w has {w.shape[1]} rows")
    x_lead = tuple(x.shape[:-2])
    idx_shape = tuple(rhsIndices.shape)
    out_lead, xm = gather_batch_maps(x_lead, idx_shape)
    x_batch = int(np.prod(x_lead)) if x_lead else 1
    batch = int(np.prod(out_lead)) if out_lead else 1
    keep = []
    x_map = None
    if xm is not None:
        x_map = DeviceArray.fromNumpy(xm, 7)
        keep.append(x_map)
    idx = rhsIndices
    if idx_shape != out_lead:
        host = np.broadcast_to(rhsIndices.rawNumpy().reshape(idx_shape), out_lead).ravel()
        idx = DeviceArray.fromNumpy(np.ascontiguousarray(host), rhsIndices.dtype)
        keep.append(idx)
    y = DeviceArray.empty(out_lead + (M, N), x.dtype)
    if sortedIndices and transpose and M == 1 and x_map is None:
        _lib.call("mlxq_gather_qmm_sorted", x.ptr, x.dtype, batch, K, idx.ptr, w.ptr, scales.ptr, biases.ptr, E, N,
                  spec.groupSize, spec.bits, y.ptr, None)
    else:
        _lib.call("mlxq_gather_qmm", x.ptr, x.dtype, x_batch, batch, M, K,
                  x_map.ptr if x_map is not None else None, idx.ptr, w.ptr, scales.ptr, biases.ptr, E, N,
                  spec.groupSize, spec.bits, int(bool(transpose)), y.ptr, None)
    # the temporaries live as long as the output: the launch (or a captured
    # graph replaying it) reads them after this returns
    y._deps = keep
    return y


# ------------------------------------------------------------------ masks

@dataclass
class Mask:
    """gemma4-base.ts Mask.  `arr` is a host bool array for "array" masks;
    `window` records createCausalMask's windowSize so the device path can
    apply the same mask without reading `arr`."""

    mode: str
    arr: Optional[np.ndarray] = None
    causalEquivalent: bool = False
    window: Optional[int] = None


def createCausalMask(N: int, offset: int, windowSize: Optional[int]) -> Mask:
    """bool [N, offset + N]: linds >= rinds (and linds < rinds + window)."""
    rinds = np.arange(offset + N)[None, :]
    linds = np.arange(offset, offset + N)[:, None]
    m = linds >= rinds
    if windowSize is not None:
        m &= linds < rinds + windowSize
    return Mask("array", m, causalEquivalent=windowSize is None, window=windowSize)


_MASK_NONE, _MASK_CAUSAL, _MASK_ARRAY = 0, 1, -1


def _mask_args(mask: Mask):
    """(mode, window) for mlxq_quantized_sdpa; _MASK_ARRAY for an array mask
    that is neither the causal matrix nor a causal window (applied as given)."""
    if mask is None or mask.mode == "":
        return _MASK_NONE, 0
    if mask.mode == "causal":
        return _MASK_CAUSAL, 0
    if mask.mode == "array":
        if mask.causalEquivalent:
            return _MASK_CAUSAL, 0
        if mask.window is not None:
            return _MASK_CAUSAL, int(mask.window)
        return _MASK_ARRAY, 0
    raise ValueError(f"unknown mask mode {mask.mode!r}")


def _array_mask(arr, B: int, L: int, n_keys: int):
    """A bool mask broadcastable to [B, 1, L, keys] (the reference's unfused
    path broadcasts it over heads: gemma4-base.ts:1320-1327) as a device uint8
    [Bm, L, N] plus its (batch, row) strides in elements."""
    if arr is None:
        raise ValueError("quantizedSdpa: array mask without an array")
    m = np.asarray(arr)
    if m.ndim == 4:
        if m.shape[1] != 1:
            raise ValueError("quantizedSdpa: array masks may not vary over heads")
        m = m[:, 0]
    if m.ndim == 2:
        m = m[None]
    if m.ndim != 3 or m.shape[0] not in (1, B) or m.shape[1] != L:
        raise ValueError(f"quantizedSdpa: mask shape {np.shape(arr)} does not broadcast to [{B}, 1, {L}, N]")
    if m.shape[2] < n_keys:
        raise ValueError(f"quantizedSdpa: mask covers {m.shape[2]} keys, the cache view has {n_keys}")
    dev = DeviceArray.fromNumpy(np.ascontiguousarray(m != 0, dtype=np.uint8), Dtype.uint8)
    return dev, (m.shape[1] * m.shape[2] if m.shape[0] > 1 else 0), m.shape[2]


def _cache_view(t: QuantizedTensor, what: str):
    """(n_kv, capacity) of a [B, H, n, .] view into a [B, H, capacity, .] buffer."""
    B, H, n, W = t.packed.shape
    caps = []
    for a in (t.packed, t.scales, t.biases):
        st = a.strides
        if st[3] != 1 or st[1] % a.shape[3] or st[0] != st[1] * H:
            raise ValueError(f"{what}: unsupported cache view layout")
        caps.append(st[1] // a.shape[3])
    if len(set(caps)) != 1:
        raise ValueError(f"{what}: packed/scales/biases capacities differ")
    return n, caps[0]


def quantizedSdpa(q: DeviceArray, kq: QuantizedTensor, vq: QuantizedTensor, scale: float, mask: Optional[Mask],
                  groupSize: int, bits: int, *, validLen: Optional[DeviceArray] = None,
                  ringOffset: Optional[DeviceArray] = None) -> DeviceArray:
    """Attention of q [B, Hq, L, D] over quantized K/V cache views
    [B, Hkv, N, .] -> [B, Hq, L, D].  `validLen` / `ringOffset` (device int32
    [B]) describe per-row windows of a batched ring cache."""
    _need_contiguous(q, "q")
    B, Hq, L, D = q.shape
    Hkv = kq.packed.shape[1]
    n_k, cap_k = _cache_view(kq, "keys")
    n_v, cap_v = _cache_view(vq, "values")
    if (n_k, cap_k) != (n_v, cap_v):
        raise ValueError("keys and values views differ")
    if kq.packed.shape[3] * 32 // bits != D:
        raise ValueError("head_dim of q and cache differ")
    mode, window = _mask_args(mask)
    out = DeviceArray.empty(q.shape, q.dtype)
    vl = validLen.ptr if validLen is not None else None
    ro = ringOffset.ptr if ringOffset is not None else None
    if mode == _MASK_ARRAY:
        dm, bstride, rstride = _array_mask(mask.arr, B, L, cap_k if validLen is not None else n_k)
        _lib.call("mlxq_quantized_sdpa_array_mask", q.ptr, q.dtype, B, Hq, Hkv, L, D,
                  kq.packed.ptr, kq.scales.ptr, kq.biases.ptr, vq.packed.ptr, vq.scales.ptr, vq.biases.ptr,
                  cap_k, n_k, vl, ro, dm.ptr, bstride, rstride, ctypes.c_float(scale), groupSize, bits, out.ptr,
                  None)
        out._deps = [dm]  # the launch (or a captured graph replaying it) reads the mask after this returns
        return out
    _lib.call("mlxq_quantized_sdpa", q.ptr, q.dtype, B, Hq, Hkv, L, D,
              kq.packed.ptr, kq.scales.ptr, kq.biases.ptr, vq.packed.ptr, vq.scales.ptr, vq.biases.ptr,
              cap_k, n_k, vl, ro, mode, window, ctypes.c_float(scale), groupSize, bits, out.ptr, None)
    return out
