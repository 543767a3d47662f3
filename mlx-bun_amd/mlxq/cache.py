"""KV caches on the device (host bookkeeping over libmlxq).

Step-for-step mirrors of the reference's QuantizedKVCache
(src/model/gemma4-base.ts:419-600) and RotatingQuantizedKVCache (:932-1260):
same growth, ring index, temporal reordering, trimming and fetched views,
so fetched triples are identical to the reference's, slot for slot.

What changes is the device work per update: new rows are quantized straight
into their cache slots by one mlxq_kv_append launch per tensor (the
reference quantizes into temporaries, then slice_update's six arrays), and
buffer reshapes (grow / trim / reorder) are strided device copies.

The T-typed caches a generation starts with, KVCache (:254-405) and
RotatingKVCache (:604-910), are mirrored too, for what the quantized path
needs of them: their buffers as laid out and their offset / ring index, which
toQuantized turns into the quantized caches above (one mlxq_quantize per
tensor over the whole buffer), and maybeQuantizeKv (src/generate.ts:101-129),
which converts a model's caches layer by layer.
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple

from . import _lib
from .array import DeviceArray, Dtype, itemsize
from .ops import Mask, QuantizedTensor, createCausalMask, quantize


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


# ------------------------------------------------------------ T-typed caches

def _write_rows(dst: DeviceArray, x: DeviceArray, pos: int) -> None:
    """dst[:, :, pos:pos+S] = x for dst a [B, H, cap, D] buffer and x a
    contiguous [B, H, S, D] array (the reference's sliceUpdate)."""
    B, H, S, D = x.shape
    isz = itemsize(x.dtype)
    _lib.call("mlxq_copy_2d", dst.ptr + pos * D * isz, dst.shape[2] * D * isz, x.ptr, S * D * isz, S * D * isz,
              B * H, None)


def _own(a: DeviceArray) -> DeviceArray:
    """A new contiguous copy of a [B, H, S, D] array or view."""
    return _concat_axis2([a])


class KVCache:
    """Growing T-typed cache (gemma4-base.ts:254-405): capacity grows by
    STEP = 256 slots (by the whole steps a chunk needs), new rows are written
    at `offset`, fetch returns the first `offset` slots."""

    STEP = 256

    def __init__(self):
        self.keys: Optional[DeviceArray] = None
        self.values: Optional[DeviceArray] = None
        self.offset = 0

    def updateAndFetch(self, k: DeviceArray, v: DeviceArray) -> Tuple[DeviceArray, DeviceArray]:
        _check_input(k, v)
        prev = self.offset
        L = k.shape[2]
        if self.keys is None or prev + L > self.keys.shape[2]:
            B, H, _, D = k.shape
            vD = v.shape[3]
            n = ((self.STEP + L - 1) // self.STEP) * self.STEP
            newK = DeviceArray.zeros((B, H, n, D), k.dtype)
            newV = DeviceArray.zeros((B, H, n, vD), v.dtype)
            if self.keys is not None:
                # an offset off a STEP boundary: the buffer is cut back to the
                # written rows before the new block is appended
                keepK = self.keys if prev % self.STEP == 0 else _cut(self.keys, 0, prev)
                keepV = self.values if prev % self.STEP == 0 else _cut(self.values, 0, prev)
                ck, cv = _concat_axis2([keepK, newK]), _concat_axis2([keepV, newV])
                for a in (self.keys, self.values, newK, newV):
                    a.dispose()
                self.keys, self.values = ck, cv
            else:
                self.keys, self.values = newK, newV
        self.offset += L
        _write_rows(self.keys, k, prev)
        _write_rows(self.values, v, prev)
        return _cut(self.keys, 0, self.offset), _cut(self.values, 0, self.offset)

    def makeMask(self, N: int, windowSize: Optional[int]) -> Mask:
        if N == 1:
            return Mask("")
        if self.offset == 0 and (windowSize is None or N <= windowSize):
            return Mask("causal")
        return createCausalMask(N, self.offset, windowSize)

    def state(self) -> List[DeviceArray]:
        return [self.keys, self.values] if self.keys is not None else []

    def isTrimmable(self) -> bool:
        return True

    def trim(self, n: int) -> None:
        self.offset = max(0, self.offset - n)

    def toQuantized(self, groupSize: int, bits: int) -> QuantizedKVCache:
        """KVCache.toQuantized (gemma4-base.ts:393-404): the whole buffer,
        padding included (it is overwritten before it is read), quantized into
        a QuantizedKVCache at the same offset; this cache is released."""
        q = QuantizedKVCache(groupSize, bits)
        q.offset = self.offset
        if self.keys is not None:
            q.keys = quantize(self.keys, groupSize, bits)
            q.values = quantize(self.values, groupSize, bits)
        self.dispose()
        return q

    def dispose(self) -> None:
        for a in (self.keys, self.values):
            if a is not None:
                a.dispose()
        self.keys = self.values = None
        self.offset = 0


class RotatingKVCache:
    """T-typed sliding-window ring of `maxSize` slots, keep = 0
    (gemma4-base.ts:604-910): S = 1 writes in place at the ring index and
    rotates at maxSize; S > 1 puts the ring in temporal order, trims it to
    the window and appends."""

    STEP = 256

    def __init__(self, maxSize: int):
        self.maxSize = maxSize
        self.keys: Optional[DeviceArray] = None
        self.values: Optional[DeviceArray] = None
        self.offset = 0
        self.ringIdx = 0

    def _seq_len(self) -> int:
        return 0 if self.keys is None else self.keys.shape[2]

    def _temporal(self, a: DeviceArray) -> DeviceArray:
        """A new buffer with the ring in temporal order (#temporalOrder)."""
        S = a.shape[2]
        if self.ringIdx == S:
            return _own(a)
        if self.ringIdx < self.offset:
            return _concat_axis2([_cut(a, self.ringIdx, S), _cut(a, 0, self.ringIdx)])
        return _own(_cut(a, 0, self.ringIdx))

    def _update_concat(self, k: DeviceArray, v: DeviceArray):
        S = k.shape[2]
        if self.keys is None:
            self.keys, self.values = _own(k), _own(v)
        else:
            tk, tv = self._temporal(self.keys), self._temporal(self.values)
            self.keys.dispose()
            self.values.dispose()
            self.ringIdx = tk.shape[2]
            trim = max(self.ringIdx - self.maxSize + 1, 0)
            self.keys = _concat_axis2([_cut(tk, trim, tk.shape[2]), k])
            self.values = _concat_axis2([_cut(tv, trim, tv.shape[2]), v])
            tk.dispose()
            tv.dispose()
        self.offset += S
        self.ringIdx = self._seq_len()
        return self._fetch_all()

    def _update_in_place(self, k: DeviceArray, v: DeviceArray):
        B, H, S, D = k.shape
        vD = v.shape[3]
        prev = self.offset
        if self.keys is None or (prev >= self._seq_len() and self._seq_len() < self.maxSize):
            new_size = min(self.STEP, self.maxSize - prev)
            newK = DeviceArray.zeros((B, H, new_size, D), k.dtype)
            newV = DeviceArray.zeros((B, H, new_size, vD), v.dtype)
            if self.keys is not None:
                ck, cv = _concat_axis2([self.keys, newK]), _concat_axis2([self.values, newV])
                for a in (self.keys, self.values, newK, newV):
                    a.dispose()
                self.keys, self.values = ck, cv
            else:
                self.keys, self.values = newK, newV
            self.ringIdx = prev
        trim = self._seq_len() - self.maxSize
        if trim > 0:
            tk = _own(_cut(self.keys, trim, self._seq_len()))
            tv = _own(_cut(self.values, trim, self._seq_len()))
            self.keys.dispose()
            self.values.dispose()
            self.keys, self.values = tk, tv
            self.ringIdx = self.maxSize
        if self.ringIdx == self.maxSize:
            self.ringIdx = 0  # rotate (keep = 0)
        _write_rows(self.keys, k, self.ringIdx)
        _write_rows(self.values, v, self.ringIdx)
        self.offset += S
        self.ringIdx += S
        if self.offset < self.maxSize:
            return _cut(self.keys, 0, self.offset), _cut(self.values, 0, self.offset)
        return self._fetch_all()

    def _fetch_all(self):
        return _cut(self.keys, 0, self._seq_len()), _cut(self.values, 0, self._seq_len())

    def updateAndFetch(self, k: DeviceArray, v: DeviceArray) -> Tuple[DeviceArray, DeviceArray]:
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
        return [self.keys, self.values] if self.keys is not None else []

    def isTrimmable(self) -> bool:
        return self.offset < self.maxSize

    def toQuantized(self, groupSize: int, bits: int) -> RotatingQuantizedKVCache:
        """RotatingKVCache.toQuantized (gemma4-base.ts:887-903): the buffer
        quantized as laid out (ring order, not temporal order), with offset
        and ring index carried over; this cache is released."""
        q = RotatingQuantizedKVCache(self.maxSize, groupSize, bits)
        if self.keys is not None:
            q.keys = quantize(self.keys, groupSize, bits)
            q.values = quantize(self.values, groupSize, bits)
        q.offset = self.offset
        q.ringIdx = self.ringIdx
        self.dispose()
        return q

    def dispose(self) -> None:
        for a in (self.keys, self.values):
            if a is not None:
                a.dispose()
        self.keys = self.values = None
        self.offset = 0
        self.ringIdx = 0


# --------------------------------------------------------- cache conversion

@dataclass
class KvQuantSpec:
    """Per-layer KV quantization (src/config.ts:74-78)."""

    layerIdx: int
    bits: int
    groupSize: int


@dataclass
class KvQuantOptions:
    """The GenerateOptions fields maybeQuantizeKv reads
    (src/generate.ts:45-54)."""

    kvBits: Optional[int] = None
    kvGroupSize: Optional[int] = None
    kvConfig: Optional[Sequence[KvQuantSpec]] = None
    quantizedKvStart: Optional[int] = None


def maybeQuantizeKv(cache: list, options: KvQuantOptions) -> None:
    """maybeQuantizeKv (src/generate.ts:101-129): replace, in place, each
    T-typed cache (KVCache or RotatingKVCache) whose offset has reached the
    start (quantizedKvStart; default 0 with a per-layer kvConfig, else 5000)
    by its quantized form.  Empty caches stay (the first prefill runs in T);
    with a kvConfig only the layers it names convert, at their bits and group
    size, otherwise every cache at kvBits and kvGroupSize (default 64).  The
    conversion streams: each layer's quantize is waited for before the next
    one starts, and toQuantized has already released that layer's T buffers,
    so the transient stays at about one layer."""
    kvConfig = list(options.kvConfig or [])
    if not options.kvBits and not kvConfig:
        return
    start = options.quantizedKvStart if options.quantizedKvStart is not None else (0 if kvConfig else 5000)
    by_layer = {e.layerIdx: e for e in kvConfig} if kvConfig else None
    for i, c in enumerate(cache):
        if not isinstance(c, (KVCache, RotatingKVCache)) or c.offset < start:
            continue
        if c.offset == 0:
            continue
        if by_layer is not None:
            e = by_layer.get(i)
            if e is None:
                continue
            cache[i] = c.toQuantized(e.groupSize, e.bits)
        else:
            cache[i] = c.toQuantized(options.kvGroupSize if options.kvGroupSize is not None else 64,
                                     options.kvBits)
        _lib.call("mlxq_synchronize", None)
