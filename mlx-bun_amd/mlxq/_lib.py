"""Loader for libmlxq.so (the gfx950 C-ABI library) and its signatures.

The library is built in-tree (``make -C mlx-bun_amd``).  There is no
fallback: if the shared object is missing or fails to load, every op raises.
Errors follow the reference's FFI contract (src/mlx/ffi.ts:277-348): a
non-zero status becomes an exception carrying the library's message.
"""
from __future__ import annotations

import ctypes
import os
import threading

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.environ.get("MLXQ_LIB", os.path.join(PKG_DIR, "libmlxq.so"))

_lib = None
_init_lock = threading.Lock()
_initialised = False

# exported symbols (include/mlxq.h), used by the ABI test
SYMBOLS = (
    "mlxq_init", "mlxq_abi_version", "mlxq_last_error", "mlxq_device_count", "mlxq_target_arch",
    "mlxq_malloc", "mlxq_free", "mlxq_memcpy_htod", "mlxq_memcpy_dtoh", "mlxq_memcpy_dtod",
    "mlxq_fill_zero", "mlxq_copy_2d", "mlxq_stream_create", "mlxq_stream_destroy", "mlxq_synchronize",
    "mlxq_event_create", "mlxq_event_destroy", "mlxq_event_record", "mlxq_event_elapsed_ms",
    "mlxq_graph_begin", "mlxq_graph_end", "mlxq_graph_launch", "mlxq_graph_destroy",
    "mlxq_workspace_reserve", "mlxq_workspace_size",
    "mlxq_quantize", "mlxq_kv_append", "mlxq_dequantize", "mlxq_embedding_gather", "mlxq_quantized_matmul",
    "mlxq_gather_qmm", "mlxq_gather_qmm_sorted",
    "mlxq_quantized_sdpa", "mlxq_quantized_sdpa_noalloc", "mlxq_quantized_sdpa_array_mask",
)


class MlxqError(RuntimeError):
    """A libmlxq call returned a non-zero status."""

    def __init__(self, op: str, status: int, message: str):
        super().__init__(f"{op} failed: {message or '(no message)'} [status {status}]")
        self.status = status


def _declare(L: ctypes.CDLL) -> None:
    P, I, I64, U64, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_uint64, ctypes.c_float
    sig = {
        "mlxq_init": [I],
        "mlxq_abi_version": [],
        "mlxq_device_count": [P],
        "mlxq_malloc": [P, U64],
        "mlxq_free": [P],
        "mlxq_memcpy_htod": [P, P, U64, P],
        "mlxq_memcpy_dtoh": [P, P, U64, P],
        "mlxq_memcpy_dtod": [P, P, U64, P],
        "mlxq_fill_zero": [P, U64, P],
        "mlxq_copy_2d": [P, U64, P, U64, U64, U64, P],
        "mlxq_stream_create": [P],
        "mlxq_stream_destroy": [P],
        "mlxq_synchronize": [P],
        "mlxq_event_create": [P],
        "mlxq_event_destroy": [P],
        "mlxq_event_record": [P, P],
        "mlxq_event_elapsed_ms": [P, P, P],
        "mlxq_graph_begin": [P],
        "mlxq_graph_end": [P, P],
        "mlxq_graph_launch": [P, P],
        "mlxq_graph_destroy": [P],
        "mlxq_workspace_reserve": [U64, P],
        "mlxq_workspace_size": [P],
        "mlxq_quantize": [P, I, I64, I64, I, I, P, P, P, P],
        "mlxq_kv_append": [P, I, I64, I64, I64, I, I, P, P, P, I64, I64, P],
        "mlxq_dequantize": [P, P, P, I, I64, I64, I, I, P, P],
        "mlxq_embedding_gather": [P, I64, P, P, P, I, I64, I64, I, I, P, P],
        "mlxq_quantized_matmul": [P, I, I64, I64, I64, P, P, P, I64, I64, I, I, I, P, P],
        "mlxq_gather_qmm": [P, I, I64, I64, I64, I64, P, P, P, P, P, I64, I64, I, I, I, P, P],
        "mlxq_gather_qmm_sorted": [P, I, I64, I64, P, P, P, P, I64, I64, I, I, P, P],
        "mlxq_quantized_sdpa": [P, I, I, I, I, I, I, P, P, P, P, P, P, I64, I64, P, P, I, I, F, I, I, P, P],
        "mlxq_quantized_sdpa_noalloc": [P, I, I, I, I, I, I, P, P, P, P, P, P, I64, I64, P, P, I, I, F, I, I, P, P],
        "mlxq_quantized_sdpa_array_mask": [P, I, I, I, I, I, I, P, P, P, P, P, P, I64, I64, P, P, P, I64, I64, F, I,
                                           I, P, P],
    }
    for name, args in sig.items():
        fn = getattr(L, name)
        fn.argtypes = args
        fn.restype = ctypes.c_int
    L.mlxq_last_error.argtypes = []
    L.mlxq_last_error.restype = ctypes.c_char_p
    L.mlxq_target_arch.argtypes = []
    L.mlxq_target_arch.restype = ctypes.c_char_p


def lib() -> ctypes.CDLL:
    """The loaded library (raises if it was not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise MlxqError("load", -1, f"{LIB_PATH} not found; build it with `make -C mlx-bun_amd`")
        _lib = ctypes.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


def call(name: str, *args) -> None:
    """Invoke an mlxq_* function and raise MlxqError on a non-zero status."""
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        msg = lib().mlxq_last_error()
        raise MlxqError(name, rc, msg.decode() if msg else "")


def ensure_init(device: int = 0) -> None:
    """mlxq_init once per process (the reference's default-stream setup)."""
    global _initialised
    if _initialised:
        return
    with _init_lock:
        if not _initialised:
            call("mlxq_init", device)
            _initialised = True


def synchronize(stream=None) -> None:
    ensure_init()
    call("mlxq_synchronize", stream)
