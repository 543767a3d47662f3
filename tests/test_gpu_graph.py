"""GPU: HIP graph capture through mlxq_graph_* stays valid across later calls.

The reference interleaves a captured decode step with prefill chunks
(src/model/compiled-decode.ts; src/generate.ts:455-470, :518-600).  Here the
decode's split-K partials live in the library workspace: a later, larger call
that grows the workspace must not free the block a captured graph still
uses, and a graph replay must keep matching the eager call.
"""
import ctypes

import numpy as np
import pytest

from conftest import assert_close

pytestmark = pytest.mark.gpu

BF16 = 12


def rng_t(O, shape, seed, scale=1.0):
    r = np.random.default_rng(seed)
    return O.round_t(r.standard_normal(shape).astype(np.float32) * scale, BF16)


def _triple(t):
    from mlxq.array import DeviceArray
    from mlxq.ops import QuantizedTensor

    return QuantizedTensor(DeviceArray.fromNumpy(t[0], 3), DeviceArray.fromNumpy(t[1], BF16),
                           DeviceArray.fromNumpy(t[2], BF16))


def _ws_size():
    from mlxq import _lib

    n = ctypes.c_uint64()
    _lib.call("mlxq_workspace_size", ctypes.byref(n))
    return n.value


def test_captured_decode_survives_workspace_growth(O, mlxq_dev):
    """Capture a 32k decode (B=1 Hq=32 Hkv=8 D=128, 4-bit), then grow the
    workspace past its size (reserve, and a split wide prefill whose fp32
    partials need tens of MB), then replay the graph three times with eager
    work in between: every replay equals the eager call bit for bit and the
    fp64 oracle within the bar.  The graph keeps the workspace block it was
    captured with; it is released with the graph."""
    from mlxq import _lib, ops
    from mlxq.array import DeviceArray

    B, Hq, Hkv, D, N = 1, 32, 8, 128, 32768
    q = rng_t(O, (B, Hq, 1, D), 1)
    kq = O.quantize(rng_t(O, (B, Hkv, N, D), 2), 64, 4, BF16)
    vq = O.quantize(rng_t(O, (B, Hkv, N, D), 3), 64, 4, BF16)
    dq, dk, dv = DeviceArray.fromFloat32(q, q.shape, BF16), _triple(kq), _triple(vq)
    out = DeviceArray.empty(q.shape, BF16)
    scale = D ** -0.5

    def decode():
        _lib.call("mlxq_quantized_sdpa", dq.ptr, BF16, B, Hq, Hkv, 1, D, dk.packed.ptr, dk.scales.ptr,
                  dk.biases.ptr, dv.packed.ptr, dv.scales.ptr, dv.biases.ptr, N, N, None, None, 0, 0,
                  ctypes.c_float(scale), 64, 4, out.ptr, None)

    decode()  # eager: sizes the workspace for the decode
    eager = out.rawNumpy()
    want = O.sdpa(q, kq, vq, scale=scale, gs=64, bits=4, dtype=BF16)
    assert_close(out.toFloat32(), want, what="eager decode", dtype=BF16)

    g = ctypes.c_void_p()
    _lib.call("mlxq_graph_begin", None)
    decode()
    _lib.call("mlxq_graph_end", None, ctypes.byref(g))
    try:
        before = _ws_size()
        _lib.call("mlxq_workspace_reserve", ctypes.c_uint64(2 * before + (1 << 20)), None)
        assert _ws_size() > 2 * before
        # a split wide prefill (keys split over workgroups: fp32 partials in the new block)
        pq = rng_t(O, (1, 16, 64, 512), 4)
        pk = O.quantize(rng_t(O, (1, 2, 2048, 512), 5), 64, 4, BF16)
        pv = O.quantize(rng_t(O, (1, 2, 2048, 512), 6), 64, 4, BF16)
        pout = ops.quantizedSdpa(DeviceArray.fromFloat32(pq, pq.shape, BF16), _triple(pk), _triple(pv), 1.0,
                                 ops.Mask("causal"), 64, 4)
        assert_close(pout.toFloat32(), O.sdpa(pq, pk, pv, scale=1.0, gs=64, bits=4, dtype=BF16, causal=True),
                     what="split wide prefill after growth", dtype=BF16)
        for rep in range(3):
            _lib.call("mlxq_fill_zero", out.ptr, out.nbytes, None)
            _lib.call("mlxq_graph_launch", g, None)
            _lib.call("mlxq_synchronize", None)
            np.testing.assert_array_equal(out.rawNumpy(), eager, err_msg=f"replay {rep}")
            decode()  # eager call between replays, on the grown workspace
            _lib.call("mlxq_synchronize", None)
            np.testing.assert_array_equal(out.rawNumpy(), eager, err_msg=f"eager after replay {rep}")
    finally:
        _lib.call("mlxq_graph_destroy", g)
    decode()
    np.testing.assert_array_equal(out.rawNumpy(), eager)


def test_workspace_cannot_grow_during_capture(mlxq_dev):
    """Growth inside a capture is refused with MLXQ_ERR_STATE and a message
    naming the way out (run the call once, or reserve, before capture)."""
    from mlxq import _lib

    L = _lib.lib()
    g = ctypes.c_void_p()
    _lib.call("mlxq_graph_begin", None)
    rc = L.mlxq_workspace_reserve(ctypes.c_uint64(_ws_size() + (64 << 20)), None)
    msg = L.mlxq_last_error().decode()
    _lib.call("mlxq_graph_end", None, ctypes.byref(g))
    _lib.call("mlxq_graph_destroy", g)
    assert rc == 4 and "captured" in msg, (rc, msg)


def test_gather_qmm_temporaries_live_with_the_output(O, mlxq_dev):
    """gatherQmm with x broadcast against the indices builds device
    temporaries (x row map, broadcast indices); they stay alive with the
    returned array, so the launch never reads freed memory, and the result
    matches per-row quantized matmuls."""
    import gc

    from mlxq import ops
    from mlxq.array import DeviceArray

    E, N, K, k = 8, 256, 512, 4
    w = O.quantize(rng_t(O, (E, N, K), 7, 0.02), 64, 4, BF16)
    x = rng_t(O, (3, 1, 1, K), 8)  # SwitchGLU's expand_dims(x, (-2, -3)) of 3 tokens
    idx = np.random.default_rng(9).integers(0, E, (3, k)).astype(np.uint32)
    t = _triple(w)
    y = ops.gatherQmm(DeviceArray.fromFloat32(x, x.shape, BF16), t.packed, t.scales, t.biases,
                      DeviceArray.fromNumpy(idx, 3), ops.QuantSpec(4, 64), sortedIndices=False)
    assert len(y._deps) == 1  # the x row map (indices already have the output's shape)
    gc.collect()
    got = y.toFloat32().reshape(3, k, N)
    for b in range(3):
        for j in range(k):
            e = idx[b, j]
            ref = O.qmm(x[b, 0], w[0][e], w[1][e], w[2][e], 64, 4, BF16)
            assert_close(got[b, j], ref[0], what=f"row {b} expert slot {j}", dtype=BF16)
