"""GPU: mlxq_quantized_sdpa_noalloc (fixed per-device scratch, no device
allocation) against mlxq_quantized_sdpa through the C ABI.

Two calls in a row on the same fixed block, the second with a smaller
input (its partials overwrite only part of what the first left), each equal
bit for bit to the allocating entry point and within the bar of the fp64
oracle; a request whose partials exceed the block fails before any launch.
"""
import ctypes

import numpy as np
import pytest

from conftest import assert_close

pytestmark = pytest.mark.gpu

BF16 = 12


def rng_t(O, shape, seed):
    r = np.random.default_rng(seed)
    return O.round_t(r.standard_normal(shape).astype(np.float32), BF16)


def _dev(O, B, Hq, Hkv, N, D, seed):
    from mlxq.array import DeviceArray

    q = rng_t(O, (B, Hq, 1, D), seed)
    kq = O.quantize(rng_t(O, (B, Hkv, N, D), seed + 1), 64, 4, BF16)
    vq = O.quantize(rng_t(O, (B, Hkv, N, D), seed + 2), 64, 4, BF16)
    up = lambda t: [DeviceArray.fromNumpy(t[0], 3), DeviceArray.fromNumpy(t[1], BF16),
                    DeviceArray.fromNumpy(t[2], BF16)]
    return q, kq, vq, DeviceArray.fromFloat32(q, q.shape, BF16), up(kq), up(vq)


def _call(L, name, dq, dk, dv, B, Hq, Hkv, Lq, D, N, scale, out, mask=0):
    return getattr(L, name)(dq.ptr, BF16, B, Hq, Hkv, Lq, D, dk[0].ptr, dk[1].ptr, dk[2].ptr, dv[0].ptr, dv[1].ptr,
                            dv[2].ptr, N, N, None, None, mask, 0, ctypes.c_float(scale), 64, 4, out.ptr, None)


def test_noalloc_decode_matches_allocating_entry_point(O, mlxq_dev):
    from mlxq import _lib
    from mlxq.array import DeviceArray

    L = _lib.lib()
    # the 32k-context decode, then a smaller one (fewer heads, chunks and dims)
    for (B, Hq, Hkv, N, D, seed) in ((1, 32, 8, 32768, 128, 1), (2, 8, 2, 5000, 256, 7)):
        q, kq, vq, dq, dk, dv = _dev(O, B, Hq, Hkv, N, D, seed)
        scale = D ** -0.5
        a, b = DeviceArray.empty(q.shape, BF16), DeviceArray.empty(q.shape, BF16)
        assert _call(L, "mlxq_quantized_sdpa_noalloc", dq, dk, dv, B, Hq, Hkv, 1, D, N, scale, a) == 0, \
            L.mlxq_last_error()
        assert _call(L, "mlxq_quantized_sdpa", dq, dk, dv, B, Hq, Hkv, 1, D, N, scale, b) == 0, L.mlxq_last_error()
        np.testing.assert_array_equal(a.rawNumpy(), b.rawNumpy(), err_msg=f"N={N} D={D}")
        want = O.sdpa(q, kq, vq, scale=scale, gs=64, bits=4, dtype=BF16)
        assert_close(a.toFloat32(), want, what=f"noalloc decode N={N} D={D}", dtype=BF16)


def test_noalloc_rejects_scratch_past_the_block(O, mlxq_dev):
    """A split D 512 prefill chunk (512 queries x 8 heads over 8192 keys)
    needs ~33 MB of partials: refused with MLXQ_ERR_UNSUPPORTED and a
    message, nothing launched."""
    from mlxq import _lib
    from mlxq.array import DeviceArray

    L = _lib.lib()
    B, Hq, Hkv, Lq, N, D = 1, 16, 2, 512, 8192, 512
    dq = DeviceArray.zeros((B, Hq, Lq, D), BF16)
    dk = [DeviceArray.zeros((B, Hkv, N, D // 8), 3), DeviceArray.zeros((B, Hkv, N, D // 64), BF16),
          DeviceArray.zeros((B, Hkv, N, D // 64), BF16)]
    out = DeviceArray.empty((B, Hq, Lq, D), BF16)
    rc = _call(L, "mlxq_quantized_sdpa_noalloc", dq, dk, dk, B, Hq, Hkv, Lq, D, N, 1.0, out, mask=1)
    msg = L.mlxq_last_error().decode()
    assert rc == 2 and "fixed block" in msg, (rc, msg)
