"""GPU: the device KV caches against the reference golden and the oracle,
and attention read straight from cache views (capacity > length)."""
import os

import numpy as np
import pytest

from conftest import GOLDEN, assert_close

pytestmark = pytest.mark.gpu

BF16 = 12


def rng_t(O, shape, seed, dtype=BF16):
    r = np.random.default_rng(seed)
    return O.round_t(r.standard_normal(shape).astype(np.float32), dtype)


def test_rotating_cache_bit_exact_vs_golden(O, mlxq_dev):
    """tests/rotating-kvq.test.ts:64-105 on the device cache: offset, ring
    index and every active (packed, scales, biases) triple bit-exact at each
    checkpoint of goldens/rotating-kvq (prefill, growth, wrap, concat over a
    wrapped ring, post-wrap decode)."""
    from mlxq.array import DeviceArray
    from mlxq.cache import RotatingQuantizedKVCache

    g = np.load(os.path.join(GOLDEN, "rotating_kvq_mechanics.npz"))
    max_size, H, D, gs, bits = (int(v) for v in g["config"])
    cache = RotatingQuantizedKVCache(max_size, gs, bits)
    cps = set(g["checkpoints"].tolist())
    for i, S in enumerate(g["step_sizes"]):
        k, v = g[f"step{i}_k"], g[f"step{i}_v"]
        qk, qv = cache.updateAndFetchQuantized(DeviceArray.fromFloat32(k, k.shape, BF16),
                                               DeviceArray.fromFloat32(v, v.shape, BF16))
        if i in cps:
            off, idx = g[f"cp{i}_offset_idx"]
            assert (cache.offset, cache.ringIdx) == (off, idx), i
            for n, t in (("k", qk), ("v", qv)):
                np.testing.assert_array_equal(t.packed.rawNumpy(), g[f"cp{i}_{n}_packed"], err_msg=f"{i}{n}")
                np.testing.assert_array_equal(t.scales.toFloat32(), g[f"cp{i}_{n}_scales"])
                np.testing.assert_array_equal(t.biases.toFloat32(), g[f"cp{i}_{n}_biases"])
    cache.dispose()


def test_quantized_cache_matches_oracle_and_feeds_sdpa(O, mlxq_dev):
    """Prefill 300 + 40 decode steps + a 1000-token chunk: fetched views equal the
    oracle cache's, and attention read in place from the views (capacity
    stride > length) matches the oracle on the same triples."""
    from mlxq import ops
    from mlxq.array import DeviceArray
    from oracle.kvcache import QuantizedKVCache as RefCache
    from mlxq.cache import QuantizedKVCache

    B, H, D, gs, bits = 1, 4, 128, 64, 4
    dev, ref = QuantizedKVCache(gs, bits), RefCache(gs, bits)
    steps = [300] + [1] * 40 + [1000]
    for i, S in enumerate(steps):
        k, v = rng_t(O, (B, H, S, D), 2 * i), rng_t(O, (B, H, S, D), 2 * i + 1)
        dk, dv = dev.updateAndFetchQuantized(DeviceArray.fromFloat32(k, k.shape, BF16),
                                             DeviceArray.fromFloat32(v, v.shape, BF16))
        rk, rv = ref.update_and_fetch(k, v, BF16)
        assert dev.offset == ref.offset
        if i in (0, 17, len(steps) - 1):
            for a, b in zip((dk.packed, dk.scales, dk.biases, dv.packed, dv.scales, dv.biases), rk + rv):
                np.testing.assert_array_equal(a.rawNumpy(), b)
    assert dev.keys.packed.shape[2] > dev.offset  # views really are strided
    q = rng_t(O, (B, 8, 1, D), 99)
    out = ops.quantizedSdpa(DeviceArray.fromFloat32(q, q.shape, BF16), dk, dv, 0.1, dev.makeMask(1, None), gs, bits)
    want = O.sdpa(q, rk, rv, scale=0.1, gs=gs, bits=bits, dtype=BF16)
    assert_close(out.toFloat32(), want, what="sdpa over cache views", dtype=BF16)
    dev.dispose()
