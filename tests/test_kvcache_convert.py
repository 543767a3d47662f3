"""The T-typed caches and their conversion to quantized caches (CPU oracle).

oracle/kvcache.py restates KVCache / RotatingKVCache
(src/model/gemma4-base.ts:254-405, :604-910), their toQuantized (:393-404,
:887-903) and maybeQuantizeKv (src/generate.ts:101-129).  What pins them:

* goldens/rotating-kvq (MLX outputs of a RotatingQuantizedKVCache driven
  through prefill, growth, wrap, a concat over the wrapped ring and post-wrap
  decode): quantize is row-wise, so a T ring driven by the same steps,
  converted at any step and driven on as a quantized ring, must land on the
  golden's triples, offset and ring index at every later checkpoint.  This
  fails if the conversion quantized the ring in temporal order, dropped the
  ring index, or if the T ring's mechanics differed from the quantized one's.
* the reference's own conversion case (tests/rotating-kvq.test.ts:107-166):
  a T ring past its wrap converted at 8 bits keeps offset / ring index, its
  dequantized ring is within 0.02 of the T values, and it decodes on.
* the growing cache: every fetch is the concatenation of what was written
  (brute force), capacities follow the STEP rule worked by hand, and a
  converted cache driven on equals a quantized cache driven from the start.
"""
import os

import numpy as np
import pytest

from conftest import GOLDEN


@pytest.fixture(scope="module")
def golden():
    return np.load(os.path.join(GOLDEN, "rotating_kvq_mechanics.npz"))


def _check_cp(O, golden, i, cache, kt, vt):
    off, idx = golden[f"cp{i}_offset_idx"]
    assert (cache.offset, cache.ring_idx) == (off, idx), f"step {i}"
    for name, t in (("k", kt), ("v", vt)):
        np.testing.assert_array_equal(t[0], golden[f"cp{i}_{name}_packed"], err_msg=f"step {i} {name}")
        np.testing.assert_array_equal(O.from_t(t[1], O.BF16), golden[f"cp{i}_{name}_scales"])
        np.testing.assert_array_equal(O.from_t(t[2], O.BF16), golden[f"cp{i}_{name}_biases"])


@pytest.mark.parametrize("convert_at", [0, 10, 16, 17, 20, 21, 25])
def test_rotating_conversion_lands_on_golden(O, golden, convert_at):
    from oracle.kvcache import RotatingKVCache

    max_size, H, D, gs, bits = (int(v) for v in golden["config"])
    cps = set(golden["checkpoints"].tolist())
    t = RotatingKVCache(max_size)
    q = None
    checked = 0
    for i, S in enumerate(golden["step_sizes"]):
        k, v = golden[f"step{i}_k"], golden[f"step{i}_v"]
        if q is None:
            t.update_and_fetch(k, v)
            if i == convert_at:
                q = t.to_quantized(gs, bits, O.BF16)
                assert (q.offset, q.ring_idx) == (t.offset, t.ring_idx)
                kt, vt = q._active()
            else:
                continue
        else:
            kt, vt = q.update_and_fetch(k, v, O.BF16)
        if i in cps:
            _check_cp(O, golden, i, q, kt, vt)
            checked += 1
    assert checked == sum(c >= convert_at for c in cps)


def test_t_ring_fetch_matches_rolled_history(O, golden):
    """The T ring's fetch, put in temporal order, is the last min(offset,
    max_size) rows written (brute force over the golden's steps)."""
    from oracle.kvcache import RotatingKVCache

    max_size = int(golden["config"][0])
    t = RotatingKVCache(max_size)
    hist = []
    for i, S in enumerate(golden["step_sizes"]):
        k = golden[f"step{i}_k"]
        fk, _ = t.update_and_fetch(k, golden[f"step{i}_v"])
        hist.append(k)
        allk = np.concatenate(hist, 2)
        n = fk.shape[2]
        if S == 1:
            # in-place: ring order; rows [ring_idx:] then [:ring_idx] are oldest first
            order = np.concatenate([fk[:, :, t.ring_idx:], fk[:, :, :t.ring_idx]], 2) if t.offset >= max_size else fk
            np.testing.assert_array_equal(order, allk[:, :, -n:])
        else:
            # concat: temporal order, the window plus the new chunk
            np.testing.assert_array_equal(fk, allk[:, :, -n:])


def test_reference_wrapped_ring_conversion_case(O):
    """tests/rotating-kvq.test.ts:107-166: MAX 64, H 2, D 64, 70 single-row
    steps of the reference LCG (seeds 100 + i / 900 + i), toQuantized(64, 8)."""
    from oracle.kvcache import RotatingKVCache

    MAX, H, D = 64, 2, 64

    def mk(seed):
        return O.round_t(O.lcg_floats(H * D, seed).reshape(1, H, 1, D), O.BF16)

    t = RotatingKVCache(MAX)
    for i in range(70):
        t.update_and_fetch(mk(100 + i), mk(900 + i))
    ring = t.keys.copy()
    off, idx = t.offset, t.ring_idx
    assert (off, idx) == (70, 6)
    q = t.to_quantized(64, 8, O.BF16)
    assert (q.offset, q.ring_idx) == (off, idx)
    assert q.keys[0].shape[2] == MAX
    deq = O.dequantize(*q.keys, 64, 8, O.BF16)
    assert np.abs(deq - ring).max() < 0.02
    qk, _ = q.update_and_fetch(mk(7777), mk(8888), O.BF16)
    assert qk[0].shape[2] == MAX and q.offset == off + 1


def test_growing_cache_capacity_and_fetch(O):
    from oracle.kvcache import KVCache

    r = np.random.default_rng(5)
    c = KVCache()
    hist = []
    # (chunk, capacity after): 300 -> 2 steps; +250 at offset 300 (off a
    # STEP boundary) cuts back to 300 and adds one step; +1 fits; +6 at 551
    # needs 557 > 556: cut back to 551, one step more
    for L, cap in ((300, 512), (250, 556), (1, 556), (6, 807)):
        k = r.standard_normal((1, 2, L, 64)).astype(np.float32)
        fk, fv = c.update_and_fetch(k, -k)
        hist.append(k)
        assert c.keys.shape[2] == cap
        np.testing.assert_array_equal(fk, np.concatenate(hist, 2))
        np.testing.assert_array_equal(fv, -np.concatenate(hist, 2))
        assert not c.keys[:, :, c.offset:].any()  # padding is zeros


def test_growing_conversion_equals_quantized_from_start(O):
    """A converted growing cache driven on equals a quantized cache that saw
    every step (same capacity, same fetched triples); the padding slots of
    the converted buffer are quantize(0) rows, not zero rows."""
    from oracle.kvcache import KVCache, QuantizedKVCache

    r = np.random.default_rng(6)
    steps = [300, 250] + [1] * 9
    xs = [(O.round_t(r.standard_normal((1, 2, L, 128)).astype(np.float32), O.BF16),
           O.round_t(r.standard_normal((1, 2, L, 128)).astype(np.float32), O.BF16)) for L in steps]
    ref = QuantizedKVCache(64, 4)
    for k, v in xs:
        rk, rv = ref.update_and_fetch(k, v, O.BF16)
    t = KVCache()
    for k, v in xs[:2]:
        t.update_and_fetch(k, v)
    q = t.to_quantized(64, 4, O.BF16)
    assert q.offset == 550 and q.keys[0].shape[2] == 556
    pad_scale = O.from_t(q.keys[1][:, :, 550:], O.BF16)
    assert np.all(pad_scale == O.round_t(np.float32(-1e-7), O.BF16))
    for k, v in xs[2:]:
        qk, qv = q.update_and_fetch(k, v, O.BF16)
    assert q.keys[0].shape[2] == ref.keys[0].shape[2]
    for a, b in zip(qk + qv, rk + rv):
        np.testing.assert_array_equal(a, b)


def test_maybe_quantize_kv_rules(O):
    """src/generate.ts:101-129: nothing without kvBits / kvConfig; empty
    caches and caches below the start stay; default start 5000 for kvBits,
    0 for kvConfig; a kvConfig converts only the layers it names."""
    from oracle.kvcache import (KVCache, QuantizedKVCache, RotatingKVCache, RotatingQuantizedKVCache,
                                maybe_quantize_kv)

    def filled(c, n):
        x = np.zeros((1, 1, n, 64), np.float32)
        if n:
            c.update_and_fetch(x, x)
        return c

    caches = [filled(KVCache(), 10), filled(RotatingKVCache(32), 40), KVCache(), filled(KVCache(), 6000), "other"]
    same = maybe_quantize_kv(caches, O.BF16)
    assert all(a is b for a, b in zip(same, caches))
    out = maybe_quantize_kv(caches, O.BF16, kv_bits=4)  # start 5000
    assert [type(c).__name__ for c in out] == ["KVCache", "RotatingKVCache", "KVCache", "QuantizedKVCache", "str"]
    out = maybe_quantize_kv(caches, O.BF16, kv_bits=8, quantized_kv_start=0)
    assert isinstance(out[0], QuantizedKVCache) and isinstance(out[1], RotatingQuantizedKVCache)
    assert isinstance(out[2], KVCache)  # empty: the first prefill runs in T
    assert out[0].bits == 8 and out[0].gs == 64
    out = maybe_quantize_kv(caches, O.BF16, kv_config={1: (4, 32)})
    assert isinstance(out[0], KVCache) and isinstance(out[1], RotatingQuantizedKVCache)
    assert (out[1].bits, out[1].gs, out[1].offset, out[1].ring_idx) == (4, 32, 40, 40)  # a 40-row first chunk is kept whole
