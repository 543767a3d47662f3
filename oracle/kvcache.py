"""Restatement of the reference's KV caches over numpy arrays.

TEST INFRASTRUCTURE ONLY (the checker for the device caches in the mlxq
package).  Pure bookkeeping around ``oracle.quantize``: growth, ring writes,
temporal reordering and trimming, step for step as
src/model/gemma4-base.ts:419-600 (QuantizedKVCache) and :932-1260
(RotatingQuantizedKVCache) do them.  A triple is (packed, scales, biases)
with shapes [B, H, S, D*bits/32], [B, H, S, D/gs] x 2 (T bit patterns).

The T-typed caches (KVCache :254-405, RotatingKVCache :604-910; values held
as float32 arrays of T values), their toQuantized conversions (:393-404,
:887-903) and maybeQuantizeKv (src/generate.ts:101-129) are restated below
the quantized ones.
"""
from __future__ import annotations

import numpy as np

from . import oracle as O


def _zeros_triple(B, H, S, D, gs, bits, dtype):
    tnp = np.float32 if dtype == O.F32 else np.uint16
    return (np.zeros((B, H, S, D * bits // 32), np.uint32),
            np.zeros((B, H, S, D // gs), tnp),
            np.zeros((B, H, S, D // gs), tnp))


def _map(t, f):
    return tuple(f(a) for a in t)


class QuantizedKVCache:
    """gemma4-base.ts:419-600: grows in STEP=256 slots, quantizes new rows and
    writes them at `offset`; fetch returns the first `offset` slots."""

    STEP = 256

    def __init__(self, group_size: int, bits: int):
        self.gs, self.bits = group_size, bits
        self.keys = self.values = None
        self.offset = 0

    def update_and_fetch(self, k, v, dtype):
        B, H, L, kD = k.shape
        vD = v.shape[3]
        prev = self.offset
        if self.keys is None or prev + L > self.keys[0].shape[2]:
            new_steps = ((self.STEP + L - 1) // self.STEP) * self.STEP
            if self.keys is not None and prev % self.STEP != 0:
                self.keys = _map(self.keys, lambda a: a[:, :, :prev])
                self.values = _map(self.values, lambda a: a[:, :, :prev])
            zk = _zeros_triple(B, H, new_steps, kD, self.gs, self.bits, dtype)
            zv = _zeros_triple(B, H, new_steps, vD, self.gs, self.bits, dtype)
            if self.keys is None:
                self.keys, self.values = zk, zv
            else:
                self.keys = tuple(np.concatenate([a, z], 2) for a, z in zip(self.keys, zk))
                self.values = tuple(np.concatenate([a, z], 2) for a, z in zip(self.values, zv))
        self.offset += L
        kq = O.quantize(k, self.gs, self.bits, dtype)
        vq = O.quantize(v, self.gs, self.bits, dtype)
        for dst, src in ((self.keys, kq), (self.values, vq)):
            for d, s in zip(dst, src):
                d[:, :, prev:self.offset] = s
        return (_map(self.keys, lambda a: a[:, :, :self.offset]),
                _map(self.values, lambda a: a[:, :, :self.offset]))


class RotatingQuantizedKVCache:
    """gemma4-base.ts:932-1260 (keep=0): ring of `max_size` slots.  S=1
    writes in place at ringIdx (#updateInPlace :1026-1094); S>1 reorders the
    ring into temporal order, trims and appends (#updateConcat :1003-1024)."""

    STEP = 256

    def __init__(self, max_size: int, group_size: int, bits: int):
        self.max_size, self.gs, self.bits = max_size, group_size, bits
        self.keys = self.values = None
        self.offset = 0
        self.ring_idx = 0

    def _seq_len(self):
        return 0 if self.keys is None else self.keys[0].shape[2]

    def _temporal(self, t):
        S = t[0].shape[2]
        if self.ring_idx == S:
            return _map(t, lambda a: a[:, :, :S].copy())
        if self.ring_idx < self.offset:
            return _map(t, lambda a: np.concatenate([a[:, :, self.ring_idx:], a[:, :, :self.ring_idx]], 2))
        return _map(t, lambda a: a[:, :, :self.ring_idx].copy())

    @staticmethod
    def _trim(trim, t, append):
        base = _map(t, lambda a: a[:, :, trim if trim > 0 else 0:])
        if append is None:
            return base
        return tuple(np.concatenate([a, b], 2) for a, b in zip(base, append))

    def _update_concat(self, k, v, dtype):
        S = k.shape[2]
        kq = O.quantize(k, self.gs, self.bits, dtype)
        vq = O.quantize(v, self.gs, self.bits, dtype)
        if self.keys is None:
            self.keys, self.values = kq, vq
        else:
            tk, tv = self._temporal(self.keys), self._temporal(self.values)
            self.ring_idx = tk[0].shape[2]
            trim = self.ring_idx - self.max_size + 1
            self.keys = self._trim(trim, tk, kq)
            self.values = self._trim(trim, tv, vq)
        self.offset += S
        self.ring_idx = self._seq_len()
        return self._active()

    def _update_in_place(self, k, v, dtype):
        B, H, S, D = k.shape
        vD = v.shape[3]
        prev = self.offset
        if self.keys is None or (prev >= self._seq_len() and self._seq_len() < self.max_size):
            new_size = min(self.STEP, self.max_size - prev)
            nk = _zeros_triple(B, H, new_size, D, self.gs, self.bits, dtype)
            nv = _zeros_triple(B, H, new_size, vD, self.gs, self.bits, dtype)
            if self.keys is None:
                self.keys, self.values = nk, nv
            else:
                self.keys = tuple(np.concatenate([a, z], 2) for a, z in zip(self.keys, nk))
                self.values = tuple(np.concatenate([a, z], 2) for a, z in zip(self.values, nv))
            self.ring_idx = prev
        trim = self._seq_len() - self.max_size
        if trim > 0:
            self.keys = self._trim(trim, self.keys, None)
            self.values = self._trim(trim, self.values, None)
            self.ring_idx = self.max_size
        if self.ring_idx == self.max_size:
            self.ring_idx = 0
        kq = O.quantize(k, self.gs, self.bits, dtype)
        vq = O.quantize(v, self.gs, self.bits, dtype)
        self.keys = tuple(a.copy() for a in self.keys)
        self.values = tuple(a.copy() for a in self.values)
        for dst, src in ((self.keys, kq), (self.values, vq)):
            for d, s in zip(dst, src):
                d[:, :, self.ring_idx:self.ring_idx + S] = s
        self.offset += S
        self.ring_idx += S
        return self._active()

    def _active(self):
        up_to = self.offset if self.offset < self.max_size else self._seq_len()
        return (_map(self.keys, lambda a: a[:, :, :up_to]),
                _map(self.values, lambda a: a[:, :, :up_to]))

    def update_and_fetch(self, k, v, dtype):
        if k.shape[2] == 1:
            return self._update_in_place(k, v, dtype)
        return self._update_concat(k, v, dtype)


# ------------------------------------------------------------ T-typed caches

class KVCache:
    """gemma4-base.ts:254-324: capacity grows by whole STEP=256 blocks; when
    `offset` is not a multiple of STEP the buffer is first cut back to it."""

    STEP = 256

    def __init__(self):
        self.keys = self.values = None
        self.offset = 0

    def update_and_fetch(self, k, v):
        prev = self.offset
        B, H, L, D = k.shape
        vD = v.shape[3]
        if self.keys is None or prev + L > self.keys.shape[2]:
            n = ((self.STEP + L - 1) // self.STEP) * self.STEP
            zk = np.zeros((B, H, n, D), np.float32)
            zv = np.zeros((B, H, n, vD), np.float32)
            if self.keys is None:
                self.keys, self.values = zk, zv
            else:
                ok, ov = self.keys, self.values
                if prev % self.STEP != 0:
                    ok, ov = ok[:, :, :prev], ov[:, :, :prev]
                self.keys = np.concatenate([ok, zk], 2)
                self.values = np.concatenate([ov, zv], 2)
        self.offset += L
        self.keys[:, :, prev:self.offset] = k
        self.values[:, :, prev:self.offset] = v
        return self.keys[:, :, :self.offset], self.values[:, :, :self.offset]

    def to_quantized(self, gs, bits, dtype):
        """:393-404 -- the whole buffer (padding included), offset kept."""
        q = QuantizedKVCache(gs, bits)
        q.offset = self.offset
        if self.keys is not None:
            q.keys = O.quantize(self.keys, gs, bits, dtype)
            q.values = O.quantize(self.values, gs, bits, dtype)
        return q


class RotatingKVCache:
    """gemma4-base.ts:604-910 with keep=0: the ring mechanics of
    RotatingQuantizedKVCache over T values."""

    STEP = 256

    def __init__(self, max_size: int):
        self.max_size = max_size
        self.keys = self.values = None
        self.offset = 0
        self.ring_idx = 0

    def _seq_len(self):
        return 0 if self.keys is None else self.keys.shape[2]

    def _temporal(self, a):
        S = a.shape[2]
        if self.ring_idx == S:
            return a[:, :, :S].copy()
        if self.ring_idx < self.offset:
            return np.concatenate([a[:, :, self.ring_idx:], a[:, :, :self.ring_idx]], 2)
        return a[:, :, :self.ring_idx].copy()

    def _update_concat(self, k, v):
        S = k.shape[2]
        if self.keys is None:
            self.keys, self.values = k.copy(), v.copy()
        else:
            tk, tv = self._temporal(self.keys), self._temporal(self.values)
            self.ring_idx = tk.shape[2]
            trim = max(self.ring_idx - self.max_size + 1, 0)
            self.keys = np.concatenate([tk[:, :, trim:], k], 2)
            self.values = np.concatenate([tv[:, :, trim:], v], 2)
        self.offset += S
        self.ring_idx = self._seq_len()
        return self.keys, self.values

    def _update_in_place(self, k, v):
        B, H, S, D = k.shape
        vD = v.shape[3]
        prev = self.offset
        if self.keys is None or (prev >= self._seq_len() and self._seq_len() < self.max_size):
            n = min(self.STEP, self.max_size - prev)
            zk = np.zeros((B, H, n, D), np.float32)
            zv = np.zeros((B, H, n, vD), np.float32)
            if self.keys is None:
                self.keys, self.values = zk, zv
            else:
                self.keys = np.concatenate([self.keys, zk], 2)
                self.values = np.concatenate([self.values, zv], 2)
            self.ring_idx = prev
        trim = self._seq_len() - self.max_size
        if trim > 0:
            self.keys = self.keys[:, :, trim:].copy()
            self.values = self.values[:, :, trim:].copy()
            self.ring_idx = self.max_size
        if self.ring_idx == self.max_size:
            self.ring_idx = 0
        self.keys[:, :, self.ring_idx:self.ring_idx + S] = k
        self.values[:, :, self.ring_idx:self.ring_idx + S] = v
        self.offset += S
        self.ring_idx += S
        if self.offset < self.max_size:
            return self.keys[:, :, :self.offset], self.values[:, :, :self.offset]
        return self.keys, self.values

    def update_and_fetch(self, k, v):
        if k.shape[2] == 1:
            return self._update_in_place(k, v)
        return self._update_concat(k, v)

    def to_quantized(self, gs, bits, dtype):
        """:887-903 -- quantized as laid out (ring order); offset and ring
        index kept."""
        q = RotatingQuantizedKVCache(self.max_size, gs, bits)
        if self.keys is not None:
            q.keys = O.quantize(self.keys, gs, bits, dtype)
            q.values = O.quantize(self.values, gs, bits, dtype)
        q.offset = self.offset
        q.ring_idx = self.ring_idx
        return q


def maybe_quantize_kv(cache, dtype, kv_bits=None, kv_group_size=None, kv_config=None, quantized_kv_start=None):
    """src/generate.ts:101-129: convert T caches whose offset reached the
    start (default 0 with a per-layer config, else 5000), skipping empty
    ones; a config {layer: (bits, group_size)} converts only the layers it
    names.  Returns the new list."""
    if not kv_bits and not kv_config:
        return list(cache)
    start = quantized_kv_start if quantized_kv_start is not None else (0 if kv_config else 5000)
    out = list(cache)
    for i, c in enumerate(cache):
        if not isinstance(c, (KVCache, RotatingKVCache)) or c.offset < start or c.offset == 0:
            continue
        if kv_config:
            if i not in kv_config:
                continue
            bits, gs = kv_config[i]
        else:
            bits, gs = kv_bits, (kv_group_size if kv_group_size is not None else 64)
        out[i] = c.to_quantized(gs, bits, dtype)
    return out
