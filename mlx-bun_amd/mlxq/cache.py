"""Quantized KV caches on the device (host bookkeeping over libmlxq).

Step-for-step mirrors of the reference's QuantizedKVCache
(src/model/gemma4-base.ts:419-600) and RotatingQuantizedKVCache (:932-1260):
same growth, ring index, temporal reordering, trimming and fetched views,
so fetched triples are identical to the reference's, slot for slot.

What changes is the device work per update: new rows are quantized straight
into their cache slots by one mlxq_kv_append launch per tensor (the
reference quantizes into temporaries, then slice_update's six arrays), and
buffer reshapes (grow / trim / reorder) are strided device copies.
"""
from __future__ import annotations

from typing import List, Optional, Tuple

from . import _lib
from .array import DeviceArray, Dtype, itemsize
from .ops import Mask, QuantizedTensor, createCausalMask


def _alloc_triple(B, H, S, D, gs, bits, dtype, zero=True) -> QuantizedTensor:
    mk = DeviceArray.zeros if zero else DeviceArray.empty
    return QuantizedTensor(mk((B, H, S, D * bits // 32), Dtype.uint32),
                           mk((B, H, S, D // gs), dtype),
                           mk((B, H, S, D // gs), dtype))


def _concat_axis2(parts: List[DeviceArray]) -> DeviceArray:
    """New contiguous [B, H, sum S_i, W] array from [B, H, S_i, W] views."""
    B, H, _, W = parts[0].shape
    dtype = parts[0].dtype
    total = sum(p.shape[2] for p in parts)
    out = DeviceArray.empty((B, H, total, W), dtype)
    isz = itemsize(dtype)
    s0 = 0
    for p in parts:
        if p.shape[2]:
            dst = out.slice((0, 0, s0, 0), (B, H, s0 + p.shape[2], W))
            _lib.call("mlxq_copy_2d", dst.ptr, total * W * isz, p.ptr, p.strides[1] * isz,
                      p.shape[2] * W * isz, B * H, None)
        s0 += p.shape[2]
    return out


def _map(t: QuantizedTensor, f) -> QuantizedTensor:
    return QuantizedTensor(f(t.packed), f(t.scales), f(t.biases))


def _cut(a: DeviceArray, lo: int, hi: int) -> DeviceArray:
    B, H, _, W = a.shape
    return a.slice((0, 0, lo, 0), (B, H, hi, W))


def _append(dst: QuantizedTensor, x: DeviceArray, pos: int, gs: int, bits: int) -> None:
    """Quantize x [B, H, S, D] into dst's slots pos..pos+S-1 (mod capacity)."""
    B, H, S, D = x.shape
    cap = dst.packed.shape[2]
    _lib.call("mlxq_kv_append", x.ptr, x.dtype, B * H, S, D, gs, bits, dst.packed.ptr, dst.scales.ptr,
              dst.biases.ptr, cap, pos, None)


def _check_input(k: DeviceArray, v: DeviceArray) -> None:
    if len(k.shape) != 4 or len(v.shape) != 4 or k.shape[:3] != v.shape[:3]:
        raise ValueError("keys/values must be [B, H, S, D] with matching B, H, S")
    if not (k.is_contiguous() and v.is_contiguous()):
        raise ValueError("keys/values must be contiguous")


class QuantizedKVCache:
    """Growing quantized cache (STEP = 256 slots)."""

    STEP = 256

    def __init__(self, groupSize: int, bits: int):
        self.groupSize, self.bits = groupSize, bits
        self.keys: Optional[QuantizedTensor] = None
        self.values: Optional[QuantizedTensor] = None
        self.offset = 0

    def updateAndFetch(self, *a):
        raise RuntimeError("QuantizedKVCache: use updateAndFetchQuantized")

    def updateAndFetchQuantized(self, k: DeviceArray, v: DeviceArray) -> Tuple[QuantizedTensor, QuantizedTensor]:
        _check_input(k, v)
        B, H, L, kD = k.shape
        vD = v.shape[3]
        prev = self.offset
        if self.keys is None or prev + L > self.keys.packed.shape[2]:
            new_steps = ((self.STEP + L - 1) // self.STEP) * self.STEP
            keep = 0 if self.keys is None else (prev if prev % self.STEP != 0 else self.keys.packed.shape[2])
            cap = keep + new_steps
            nk = _alloc_triple(B, H, cap, kD, self.groupSize, self.bits, k.dtype)
            nv = _alloc_triple(B, H, cap, vD, self.groupSize, self.bits, v.dtype)
            if self.keys is not None:
                if keep:
                    for dst, src in ((nk, self.keys), (nv, self.values)):
                        for d, s in zip((dst.packed, dst.scales, dst.biases), (src.packed, src.scales, src.biases)):
                            _copy_into(d, s, keep)
                self.keys.dispose()
                self.values.dispose()
            self.keys, self.values = nk, nv
        _append(self.keys, k, prev, self.groupSize, self.bits)
        _append(self.values, v, prev, self.groupSize, self.bits)
        self.offset += L
        return self._fetch()

    def _fetch(self):
        n = self.offset
        return _map(self.keys, lambda a: _cut(a, 0, n)), _map(self.values, lambda a: _cut(a, 0, n))

    def makeMask(self, N: int, windowSize: Optional[int]) -> Mask:
        if N == 1:
            return Mask("")
        if self.offset == 0 and (windowSize is None or N <= windowSize):
            return Mask("causal")
        return createCausalMask(N, self.offset, windowSize)

    def state(self) -> List[DeviceArray]:
        if self.keys is None:
            return []
        return [self.keys.packed, self.keys.scales, self.keys.biases,
                self.values.packed, self.values.scales, self.values.biases]

    def trim(self, n: int) -> None:
        self.offset = max(0, self.offset - n)

    def dispose(self) -> None:
        for t in (self.keys, self.values):
            if t is not None:
                t.dispose()
        self.keys = self.values = None
        self.offset = 0


def _copy_into(dst_full: DeviceArray, src: DeviceArray, n: int) -> None:
    """dst_full[:, :, :n] = src[:, :, :n] (both [B, H, ., W] buffers or views)."""
    B, H, _, W = dst_full.shape
    isz = itemsize(dst_full.dtype)
    _lib.call("mlxq_copy_2d", dst_full.ptr, dst_full.strides[1] * isz, src.ptr, src.strides[1] * isz,
              n * W * isz, B * H, None)


class RotatingQuantizedKVCache:
    """Sliding-window ring of `maxSize` quantized slots (keep = 0)."""

    STEP = 256

    def __init__(self, maxSize: int, groupSize: int, bits: int):
        self.maxSize, self.groupSize, self.bits = maxSize, groupSize, bits
        self.keys: Optional[QuantizedTensor] = None
        self.values: Optional[QuantizedTensor] = None
        self.offset = 0
        self.ringIdx = 0

    def updateAndFetch(self, *a):
        raise RuntimeError("RotatingQuantizedKVCache: use updateAndFetchQuantized")

    def _seq_len(self) -> int:
        return 0 if self.keys is None else self.keys.packed.shape[2]

    def _replace(self, keys: QuantizedTensor, values: QuantizedTensor) -> None:
        for t in (self.keys, self.values):
            if t is not None:
                t.dispose()
        self.keys, self.values = keys, values

    def _temporal(self, t: QuantizedTensor) -> QuantizedTensor:
        S = t.packed.shape[2]
        if self.ringIdx == S:
            return _map(t, lambda a: _concat_axis2([_cut(a, 0, S)]))
        if self.ringIdx < self.offset:
            return _map(t, lambda a: _concat_axis2([_cut(a, self.ringIdx, S), _cut(a, 0, self.ringIdx)]))
        return _map(t, lambda a: _concat_axis2([_cut(a, 0, self.ringIdx)]))

    def _update_concat(self, k: DeviceArray, v: DeviceArray):
        B, H, S, D = k.shape
        vD = v.shape[3]
        kq = _alloc_triple(B, H, S, D, self.groupSize, self.bits, k.dtype, zero=False)
        vq = _alloc_triple(B, H, S, vD, self.groupSize, self.bits, v.dtype, zero=False)
        _append(kq, k, 0, self.groupSize, self.bits)
        _append(vq, v, 0, self.groupSize, self.bits)
        if self.keys is None:
            self._replace(kq, vq)
        else:
            tk, tv = self._temporal(self.keys), self._temporal(self.values)
            self.ringIdx = tk.packed.shape[2]
            trim = max(self.ringIdx - self.maxSize + 1, 0)

            def join(t, new):
                return QuantizedTensor(*(_concat_axis2([_cut(a, trim, a.shape[2]), n])
                                         for a, n in ((t.packed, new.packed), (t.scales, new.scales),
                                                      (t.biases, new.biases))))

            nk, nv = join(tk, kq), join(tv, vq)
            for t in (tk, tv, kq, vq):
                t.dispose()
            self._replace(nk, nv)
        self.offset += S
        self.ringIdx = self._seq_len()
        return self._active()

    def _update_in_place(self, k: DeviceArray, v: DeviceArray):
        B, H, S, D = k.shape
        vD = v.shape[3]
        prev = self.offset
        if self.keys is None or (prev >= self._seq_len() and self._seq_len() < self.maxSize):
            new_size = min(self.STEP, self.maxSize - prev)
            nk = _alloc_triple(B, H, new_size, D, self.groupSize, self.bits, k.dtype)
            nv = _alloc_triple(B, H, new_size, vD, self.groupSize, self.bits, v.dtype)
            if self.keys is None:
                self._replace(nk, nv)
            else:
                gk = QuantizedTensor(*(_concat_axis2([a, n]) for a, n in zip(
                    (self.keys.packed, self.keys.scales, self.keys.biases), (nk.packed, nk.scales, nk.biases))))
                gv = QuantizedTensor(*(_concat_axis2([a, n]) for a, n in zip(
                    (self.values.packed, self.values.scales, self.values.biases),
                    (nv.packed, nv.scales, nv.biases))))
                nk.dispose()
                nv.dispose()
                self._replace(gk, gv)
            self.ringIdx = prev
        trim = self._seq_len() - self.maxSize
        if trim > 0:
            tk = _map(self.keys, lambda a: _concat_axis2([_cut(a, trim, a.shape[2])]))
            tv = _map(self.values, lambda a: _concat_axis2([_cut(a, trim, a.shape[2])]))
            self._replace(tk, tv)
            self.ringIdx = self.maxSize
        if self.ringIdx == self.maxSize:
            self.ringIdx = 0
        _append(self.keys, k, self.ringIdx, self.groupSize, self.bits)
        _append(self.values, v, self.ringIdx, self.groupSize, self.bits)
        self.offset += S
        self.ringIdx += S
        return self._active()

    def _active(self):
        up_to = self.offset if self.offset < self.maxSize else self._seq_len()
        return _map(self.keys, lambda a: _cut(a, 0, up_to)), _map(self.values, lambda a: _cut(a, 0, up_to))

    def updateAndFetchQuantized(self, k: DeviceArray, v: DeviceArray):
        _check_input(k, v)
        return self._update_in_place(k, v) if k.shape[2] == 1 else self._update_concat(k, v)

    def makeMask(self, N: int, windowSize: Optional[int]) -> Mask:
        window = windowSize if windowSize is not None else self.maxSize
        if N > 1:
            offset = min(self.maxSize - 1, self.offset)
            if offset + N > window:
                return createCausalMask(N, offset, window)
            return Mask("causal")
        return Mask("")

    def state(self) -> List[DeviceArray]:
        if self.keys is None:
            return []
        return [self.keys.packed, self.keys.scales, self.keys.biases,
                self.values.packed, self.values.scales, self.values.biases]

    def dispose(self) -> None:
        self._replace(None, None)
        self.offset = 0
        self.ringIdx = 0
