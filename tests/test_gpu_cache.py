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


def _triples_equal(dev_t, ref_t, what):
    for a, b in zip((dev_t.packed, dev_t.scales, dev_t.biases), ref_t):
        np.testing.assert_array_equal(a.rawNumpy(), b, err_msg=what)


def test_device_ring_conversion_lands_on_golden(O, mlxq_dev):
    """The device T ring driven by the golden's steps, converted by
    toQuantized right after its wrap (step 17) and driven on as a quantized
    ring, lands bit-exact on goldens/rotating-kvq at every later checkpoint
    (src/model/gemma4-base.ts:887-903: quantized as laid out, ring index
    kept)."""
    from mlxq.array import DeviceArray
    from mlxq.cache import RotatingKVCache

    g = np.load(os.path.join(GOLDEN, "rotating_kvq_mechanics.npz"))
    max_size, H, D, gs, bits = (int(v) for v in g["config"])
    cps = set(g["checkpoints"].tolist())
    t, q = RotatingKVCache(max_size), None
    seen = 0
    for i, S in enumerate(g["step_sizes"]):
        k = DeviceArray.fromFloat32(g[f"step{i}_k"], g[f"step{i}_k"].shape, BF16)
        v = DeviceArray.fromFloat32(g[f"step{i}_v"], g[f"step{i}_v"].shape, BF16)
        if q is None:
            fk, fv = t.updateAndFetch(k, v)
            if i == 17:
                off, idx = t.offset, t.ringIdx
                q = t.toQuantized(gs, bits)
                assert (q.offset, q.ringIdx) == (off, idx) == (65, 1)
                assert t.keys is None
            continue
        qk, qv = q.updateAndFetchQuantized(k, v)
        if i in cps:
            off, idx = g[f"cp{i}_offset_idx"]
            assert (q.offset, q.ringIdx) == (off, idx), i
            for n, tt in (("k", qk), ("v", qv)):
                np.testing.assert_array_equal(tt.packed.rawNumpy(), g[f"cp{i}_{n}_packed"], err_msg=f"{i}{n}")
                np.testing.assert_array_equal(tt.scales.toFloat32(), g[f"cp{i}_{n}_scales"])
                np.testing.assert_array_equal(tt.biases.toFloat32(), g[f"cp{i}_{n}_biases"])
            seen += 1
    assert seen == 4
    q.dispose()


def test_reference_wrapped_ring_conversion_on_device(O, mlxq_dev):
    """tests/rotating-kvq.test.ts:107-166 on the device caches: MAX 64, H 2,
    D 64, 70 single-row steps of the reference LCG, toQuantized(64, 8) keeps
    offset / ring index, the dequantized ring is within 0.02 of the T ring
    (and bit-exact against the oracle's conversion), and it decodes on."""
    from mlxq import ops
    from mlxq.array import DeviceArray
    from mlxq.cache import RotatingKVCache
    from oracle.kvcache import RotatingKVCache as RefRing

    MAX, H, D = 64, 2, 64

    def mk(seed):
        return O.round_t(O.lcg_floats(H * D, seed).reshape(1, H, 1, D), O.BF16)

    t, ref = RotatingKVCache(MAX), RefRing(MAX)
    for i in range(70):
        k, v = mk(100 + i), mk(900 + i)
        t.updateAndFetch(DeviceArray.fromFloat32(k, k.shape, BF16), DeviceArray.fromFloat32(v, v.shape, BF16))
        ref.update_and_fetch(k, v)
    ring = t.keys.toFloat32()
    np.testing.assert_array_equal(ring, ref.keys)
    q, rq = t.toQuantized(64, 8), ref.to_quantized(64, 8, O.BF16)
    assert (q.offset, q.ringIdx) == (rq.offset, rq.ring_idx) == (70, 6)
    assert q.keys.packed.shape[2] == MAX
    _triples_equal(q.keys, rq.keys, "converted keys")
    _triples_equal(q.values, rq.values, "converted values")
    deq = ops.dequantize(q.keys.packed, q.keys.scales, q.keys.biases, ops.QuantSpec(8, 64)).toFloat32()
    assert np.abs(deq - ring).max() < 0.02
    k, v = mk(7777), mk(8888)
    qk, _ = q.updateAndFetchQuantized(DeviceArray.fromFloat32(k, k.shape, BF16),
                                      DeviceArray.fromFloat32(v, v.shape, BF16))
    assert qk.packed.shape[2] == MAX and q.offset == 71
    q.dispose()


def test_maybe_quantize_kv_then_decode(O, mlxq_dev):
    """maybeQuantizeKv (src/generate.ts:101-129) over a model's caches: a
    growing cache filled off a 256 boundary (300 + 250 rows: capacity 556),
    a 512-slot ring filled past its wrap (300 + 250 single rows), an empty
    cache and one below quantizedKvStart.  The two filled ones convert
    (bit-exact against the oracle's conversion, whole buffers), the others
    stay; then 5 decode steps run through the quantized caches, their fetched
    triples bit-exact against the oracle caches and attention over them
    within the bar of the fp64 oracle."""
    from mlxq import ops
    from mlxq.array import DeviceArray
    from mlxq.cache import (KVCache, KvQuantOptions, QuantizedKVCache, RotatingKVCache,
                            RotatingQuantizedKVCache, maybeQuantizeKv)
    from oracle import kvcache as R

    B, Hkv, Hq, D, gs, bits = 1, 2, 8, 128, 64, 4
    dev = [KVCache(), RotatingKVCache(512), KVCache(), KVCache()]
    ref = [R.KVCache(), R.RotatingKVCache(512), R.KVCache(), R.KVCache()]
    plan = {0: [300, 250], 1: [300] + [1] * 250, 3: [50]}
    seed = 0
    for li, steps in plan.items():
        for S in steps:
            k, v = rng_t(O, (B, Hkv, S, D), seed), rng_t(O, (B, Hkv, S, D), seed + 1)
            seed += 2
            fk, fv = dev[li].updateAndFetch(DeviceArray.fromFloat32(k, k.shape, BF16),
                                            DeviceArray.fromFloat32(v, v.shape, BF16))
            rk, rv = ref[li].update_and_fetch(k, v)
        np.testing.assert_array_equal(fk.toFloat32(), rk)
        np.testing.assert_array_equal(fv.toFloat32(), rv)
    assert dev[0].keys.shape[2] == 556 and dev[0].offset == 550
    assert (dev[1].offset, dev[1].ringIdx, dev[1].keys.shape[2]) == (550, 38, 512)
    maybeQuantizeKv(dev, KvQuantOptions(kvBits=bits, kvGroupSize=gs, quantizedKvStart=100))
    ref = R.maybe_quantize_kv(ref, O.BF16, kv_bits=bits, kv_group_size=gs, quantized_kv_start=100)
    assert [type(c).__name__ for c in dev] == ["QuantizedKVCache", "RotatingQuantizedKVCache", "KVCache", "KVCache"]
    assert isinstance(dev[0], QuantizedKVCache) and isinstance(dev[1], RotatingQuantizedKVCache)
    assert (dev[1].offset, dev[1].ringIdx) == (550, 38)
    for li in (0, 1):
        _triples_equal(dev[li].keys, ref[li].keys, f"layer {li} keys")
        _triples_equal(dev[li].values, ref[li].values, f"layer {li} values")
    for step in range(5):
        for li in (0, 1):
            k, v = rng_t(O, (B, Hkv, 1, D), 1000 + 4 * step + 2 * li), rng_t(O, (B, Hkv, 1, D), 1001 + 4 * step + 2 * li)
            qk, qv = dev[li].updateAndFetchQuantized(DeviceArray.fromFloat32(k, k.shape, BF16),
                                                     DeviceArray.fromFloat32(v, v.shape, BF16))
            rk, rv = ref[li].update_and_fetch(k, v, O.BF16)
            _triples_equal(qk, rk, f"step {step} layer {li} keys")
            _triples_equal(qv, rv, f"step {step} layer {li} values")
            q = rng_t(O, (B, Hq, 1, D), 2000 + step)
            out = ops.quantizedSdpa(DeviceArray.fromFloat32(q, q.shape, BF16), qk, qv, 1.0,
                                    dev[li].makeMask(1, None), gs, bits)
            want = O.sdpa(q, rk, rv, scale=1.0, gs=gs, bits=bits, dtype=BF16)
            assert_close(out.toFloat32(), want, what=f"decode step {step} layer {li}", dtype=BF16)
    for c in dev:
        c.dispose()
