"""GPU: argument validation at the C ABI.  Every entry point returns a status
(MLXQ_ERR_ARGUMENT for a rejected shape / dtype / size) and records a
message, the contract of the reference's mlx-c FFI (src/mlx/ffi.ts:277-348:
status per call, message surfaced as the JS Error).  No bad request reaches
a kernel; empty requests succeed without touching memory."""
import ctypes

import numpy as np
import pytest

from mlxq import _lib
from mlxq.array import DeviceArray

pytestmark = pytest.mark.gpu

OK, ARG = 0, 1
U32, I32, F16, F32, BF16 = 3, 7, 9, 10, 12


def expect(rc_and_msg, code, fragment):
    rc, msg = rc_and_msg
    assert rc == code, (rc, msg)
    assert fragment in msg, msg


def call(name, *args):
    L = _lib.lib()
    rc = getattr(L, name)(*args)
    m = L.mlxq_last_error()
    return rc, (m.decode() if m else "")


@pytest.fixture(scope="module")
def bufs(mlxq_dev):
    """One generous device buffer reused as every operand (the calls below
    are rejected or empty, so nothing is read or written)."""
    a = DeviceArray.empty((1 << 20,), U32)
    return a


def test_quantize_rejects(bufs):
    p = bufs.ptr
    expect(call("mlxq_quantize", p, BF16, 4, 128, 64, 3, p, p, p, None), ARG, "bits")
    expect(call("mlxq_quantize", p, BF16, 4, 128, 48, 4, p, p, p, None), ARG, "group_size")
    expect(call("mlxq_quantize", p, BF16, 4, 96, 64, 4, p, p, p, None), ARG, "multiple")
    expect(call("mlxq_quantize", p, 3, 4, 128, 64, 4, p, p, p, None), ARG, "dtype")
    expect(call("mlxq_quantize", None, BF16, 4, 128, 64, 4, p, p, p, None), ARG, "null")
    assert call("mlxq_quantize", None, BF16, 0, 128, 64, 4, None, None, None, None)[0] == OK  # empty


def test_kv_append_rejects(bufs):
    p = bufs.ptr
    expect(call("mlxq_kv_append", p, BF16, 2, 9, 128, 64, 4, p, p, p, 8, 0, None), ARG, "slots")
    expect(call("mlxq_kv_append", p, BF16, 2, 1, 128, 64, 4, p, p, p, 0, 0, None), ARG, "capacity")
    expect(call("mlxq_kv_append", p, BF16, 2, 1, 128, 64, 4, p, p, p, 8, -1, None), ARG, "negative")


def test_quantized_matmul_rejects(bufs):
    p = bufs.ptr
    expect(call("mlxq_quantized_matmul", p, BF16, 3, 1, 256, p, p, p, 2, 64, 64, 4, 1, p, None), ARG, "w_batch")
    expect(call("mlxq_quantized_matmul", p, BF16, 1, 1, 200, p, p, p, 1, 64, 64, 4, 1, p, None), ARG, "multiple")
    expect(call("mlxq_quantized_matmul", p, BF16, 1, 1, 256, p, p, p, 1, 64, 64, 5, 1, p, None), ARG, "bits")
    expect(call("mlxq_quantized_matmul", None, BF16, 1, 1, 256, p, p, p, 1, 64, 64, 4, 1, p, None), ARG, "null")
    expect(call("mlxq_quantized_matmul", p, BF16, -1, 1, 256, p, p, p, 1, 64, 64, 4, 1, p, None), ARG, "negative")
    assert call("mlxq_quantized_matmul", None, BF16, 0, 1, 256, None, None, None, 1, 64, 64, 4, 1, None,
                None)[0] == OK


def test_gather_qmm_rejects(bufs):
    p = bufs.ptr
    expect(call("mlxq_gather_qmm", p, BF16, 2, 4, 1, 256, None, p, p, p, p, 4, 64, 64, 4, 1, p, None), ARG, "x_map")
    expect(call("mlxq_gather_qmm", p, BF16, 1, 4, 1, 256, p, p, p, p, p, 0, 64, 64, 4, 1, p, None), ARG, "n_experts")
    expect(call("mlxq_gather_qmm", p, BF16, 1, 4, 1, 256, p, None, p, p, p, 4, 64, 64, 4, 1, p, None), ARG, "null")


def test_embedding_gather_rejects(bufs):
    p = bufs.ptr
    expect(call("mlxq_embedding_gather", None, 4, p, p, p, BF16, 100, 128, 64, 4, p, None), ARG, "null ids")
    expect(call("mlxq_embedding_gather", p, 4, p, p, p, BF16, 100, 100, 64, 4, p, None), ARG, "multiple")
    assert call("mlxq_embedding_gather", None, 0, None, None, None, BF16, 100, 128, 64, 4, None, None)[0] == OK


def test_sdpa_rejects(bufs):
    p = bufs.ptr
    f = ctypes.c_float(1.0)
    base = dict(q=p, dtype=BF16, B=1, Hq=8, Hkv=2, Lq=1, D=128, kp=p, ks=p, kb=p, vp=p, vs=p, vb=p, cap=64, n_kv=64,
                vl=None, ro=None, mask=0, window=0, scale=f, gs=64, bits=4, out=p)

    def sdpa(**kw):
        a = dict(base, **kw)
        return call("mlxq_quantized_sdpa", a["q"], a["dtype"], a["B"], a["Hq"], a["Hkv"], a["Lq"], a["D"], a["kp"],
                    a["ks"], a["kb"], a["vp"], a["vs"], a["vb"], a["cap"], a["n_kv"], a["vl"], a["ro"], a["mask"],
                    a["window"], a["scale"], a["gs"], a["bits"], a["out"], None)

    expect(sdpa(Hq=6, Hkv=4), ARG, "multiple of kv heads")
    expect(sdpa(D=1024), ARG, "head_dim")
    expect(sdpa(n_kv=65), ARG, "n_kv")
    expect(sdpa(ro=p), ARG, "ring_offset requires valid_len")
    expect(sdpa(mask=7), ARG, "mask")
    expect(sdpa(window=-1), ARG, "window")
    expect(sdpa(q=p + 2), ARG, "aligned")
    expect(sdpa(vp=None), ARG, "null")
    expect(sdpa(cap=0), ARG, "kv_capacity")
    assert sdpa(B=0)[0] == OK


def test_error_message_is_per_thread(bufs):
    """mlxq_last_error is thread-local: a failure on one thread does not
    overwrite another thread's message."""
    import threading

    p = bufs.ptr
    call("mlxq_quantize", p, BF16, 4, 128, 64, 3, p, p, p, None)
    seen = {}

    def other():
        seen["rc"] = call("mlxq_quantize", p, BF16, 4, 128, 48, 4, p, p, p, None)

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert "group_size" in seen["rc"][1]
    assert "bits" in _lib.lib().mlxq_last_error().decode()
