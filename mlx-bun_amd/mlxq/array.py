"""Device arrays for the host mirror: a device buffer plus shape and dtype.

Mirrors the part of the reference's MlxArray the hot path uses
(src/mlx/array.ts:49-237): explicit ``dispose()`` with a finalizer backstop,
``fromFloat32`` / ``toFloat32`` / ``rawBytes`` transfers and axis slicing.
Slices along an axis of a contiguous array are views sharing the owner's
buffer (``offset`` in bytes, ``strides`` in elements) -- the cache classes
hand out such views exactly as the reference's fetch does.
"""
from __future__ import annotations

import ctypes
import weakref

import numpy as np

from . import _lib


class Dtype:
    """mlx_dtype enum values (src/mlx/ffi.ts:297-300)."""

    bool_ = 0
    uint8 = 1
    uint16 = 2
    uint32 = 3
    uint64 = 4
    int8 = 5
    int16 = 6
    int32 = 7
    int64 = 8
    float16 = 9
    float32 = 10
    float64 = 11
    bfloat16 = 12


_NP_STORAGE = {Dtype.bool_: np.uint8, Dtype.uint8: np.uint8, Dtype.uint16: np.uint16, Dtype.uint32: np.uint32,
               Dtype.uint64: np.uint64, Dtype.int8: np.int8, Dtype.int16: np.int16, Dtype.int32: np.int32,
               Dtype.int64: np.int64, Dtype.float16: np.uint16, Dtype.float32: np.float32,
               Dtype.float64: np.float64, Dtype.bfloat16: np.uint16}
_ITEMSIZE = {d: np.dtype(t).itemsize for d, t in _NP_STORAGE.items()}


def itemsize(dtype: int) -> int:
    return _ITEMSIZE[dtype]


# ---------------------------------------------------------------- host T

def f32_to_bits(x, dtype: int) -> np.ndarray:
    """float32 values -> storage array of `dtype` (round-to-nearest-even)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if dtype == Dtype.float32:
        return x
    if dtype == Dtype.float16:
        with np.errstate(over="ignore"):  # out-of-range values become inf, as in MLX
            return x.astype(np.float16).view(np.uint16)
    if dtype == Dtype.bfloat16:
        u = x.view(np.uint32).astype(np.uint64)
        r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
        nan = (u & 0x7FFFFFFF) > 0x7F800000
        if nan.any():
            r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
        return r
    raise ValueError(f"not a float dtype: {dtype}")


def bits_to_f32(b, dtype: int) -> np.ndarray:
    """storage array of `dtype` -> float32."""
    if dtype == Dtype.float32:
        return np.asarray(b, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.uint16)
    if dtype == Dtype.float16:
        return b.view(np.float16).astype(np.float32)
    if dtype == Dtype.bfloat16:
        return (b.astype(np.uint32) << 16).view(np.float32)
    raise ValueError(f"not a float dtype: {dtype}")


class _Buffer:
    """Owns one device allocation; freed by dispose() or the finalizer."""

    def __init__(self, nbytes: int):
        _lib.ensure_init()
        p = ctypes.c_void_p()
        _lib.call("mlxq_malloc", ctypes.byref(p), max(int(nbytes), 1))
        self.ptr = p.value
        self.nbytes = int(nbytes)
        self._fin = weakref.finalize(self, _Buffer._free, self.ptr)

    @staticmethod
    def _free(ptr):
        try:
            _lib.lib().mlxq_free(ptr)
        except Exception:  # interpreter shutdown
            pass

    def free(self):
        self._fin()
        self.ptr = None  # any later use raises instead of touching freed memory


class DeviceArray:
    """A (possibly strided) view of a device buffer."""

    def __init__(self, buf: _Buffer, shape, dtype: int, offset: int = 0, strides=None):
        self._buf = buf
        self.shape = tuple(int(s) for s in shape)
        self.dtype = dtype
        self.offset = int(offset)
        self.strides = tuple(strides) if strides is not None else _contig_strides(self.shape)

    # -- construction -----------------------------------------------------
    @staticmethod
    def empty(shape, dtype: int) -> "DeviceArray":
        n = int(np.prod(shape)) if len(shape) else 1
        return DeviceArray(_Buffer(n * itemsize(dtype)), shape, dtype)

    @staticmethod
    def zeros(shape, dtype: int) -> "DeviceArray":
        a = DeviceArray.empty(shape, dtype)
        _lib.call("mlxq_fill_zero", a.ptr, a.nbytes, None)
        return a

    @staticmethod
    def fromNumpy(storage: np.ndarray, dtype: int) -> "DeviceArray":
        """Upload a host array already in `dtype`'s storage representation."""
        storage = np.ascontiguousarray(storage, dtype=_NP_STORAGE[dtype])
        a = DeviceArray.empty(storage.shape, dtype)
        _lib.call("mlxq_memcpy_htod", a.ptr, storage.ctypes.data_as(ctypes.c_void_p), storage.nbytes, None)
        return a

    @staticmethod
    def fromFloat32(data, shape, dtype: int = Dtype.float32) -> "DeviceArray":
        """MlxArray.fromFloat32 (+ astype): float values rounded to `dtype`."""
        x = np.asarray(data, dtype=np.float32).reshape(shape)
        return DeviceArray.fromNumpy(f32_to_bits(x, dtype), dtype)

    # -- properties ---------------------------------------------------------
    @property
    def ptr(self) -> int:
        if self._buf.ptr is None:
            raise ValueError("use of a disposed DeviceArray")
        return self._buf.ptr + self.offset

    @property
    def size(self) -> int:
        return int(np.prod(self.shape)) if self.shape else 1

    @property
    def nbytes(self) -> int:
        return self.size * itemsize(self.dtype)

    def is_contiguous(self) -> bool:
        return self.strides == _contig_strides(self.shape)

    # -- transfers ------------------------------------------------------------
    def rawNumpy(self) -> np.ndarray:
        """Storage representation on the host (a contiguous copy)."""
        dt = _NP_STORAGE[self.dtype]
        if self.is_contiguous():
            out = np.empty(self.shape, dtype=dt)
            _lib.call("mlxq_memcpy_dtoh", out.ctypes.data_as(ctypes.c_void_p), self.ptr, out.nbytes, None)
            return out
        # strided view: copy the spanned region and slice on the host
        span = _span_elems(self.shape, self.strides)
        flat = np.empty(span, dtype=dt)
        _lib.call("mlxq_memcpy_dtoh", flat.ctypes.data_as(ctypes.c_void_p), self.ptr, flat.nbytes, None)
        return np.lib.stride_tricks.as_strided(
            flat, self.shape, tuple(s * flat.itemsize for s in self.strides)).copy()

    def rawBytes(self) -> bytes:
        return self.rawNumpy().tobytes()

    def toFloat32(self) -> np.ndarray:
        return bits_to_f32(self.rawNumpy(), self.dtype)

    # -- views ------------------------------------------------------------------
    def slice(self, start, stop) -> "DeviceArray":
        """a[start:stop] per axis, as a view (MlxArray.slice)."""
        off = self.offset
        shape = []
        for ax, (a, b) in enumerate(zip(start, stop)):
            if not (0 <= a <= b <= self.shape[ax]):
                raise ValueError(f"slice {start}:{stop} out of range for shape {self.shape}")
            off += a * self.strides[ax] * itemsize(self.dtype)
            shape.append(b - a)
        return DeviceArray(self._buf, shape, self.dtype, off, self.strides)

    def dispose(self) -> None:
        """Release the device buffer (shared by every view of it)."""
        self._buf.free()

    def __repr__(self):
        return f"DeviceArray(shape={self.shape}, dtype={self.dtype})"


def _contig_strides(shape):
    st, acc = [], 1
    for s in reversed(shape):
        st.append(acc)
        acc *= s
    return tuple(reversed(st))


def _span_elems(shape, strides):
    if any(s == 0 for s in shape):
        return 0
    return 1 + sum((s - 1) * st for s, st in zip(shape, strides))
