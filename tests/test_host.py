"""Host-side logic of the mlxq mirror (CPU): T conversions, masks and the
mask/dispatch rules of the reference's caches."""
import numpy as np
import pytest

from mlxq import ops
from mlxq.array import Dtype, bits_to_f32, f32_to_bits
from mlxq.cache import QuantizedKVCache, RotatingQuantizedKVCache


@pytest.mark.parametrize("dtype", [Dtype.bfloat16, Dtype.float16])
def test_host_rounding_matches_oracle(O, dtype):
    r = np.random.default_rng(0)
    x = np.concatenate([r.standard_normal(20000).astype(np.float32) * 10.0 ** r.integers(-6, 6, 20000),
                        np.array([0.0, -0.0, np.inf, -np.inf, 65504, 65520, 1e-8, 3.0e38, -3.4e38], np.float32)])
    # exact ties of the target format
    x = np.concatenate([x, (np.arange(1, 200, dtype=np.float32) + 0.5) * 2.0 ** -7 + 1.0])
    np.testing.assert_array_equal(f32_to_bits(x, dtype), O.to_t(x, dtype))
    b = O.to_t(x, dtype)
    np.testing.assert_array_equal(bits_to_f32(b, dtype), O.from_t(b, dtype))


def test_create_causal_mask_brute_force():
    for N, off, win in [(4, 0, None), (3, 5, None), (6, 10, 4), (1, 7, 3)]:
        m = ops.createCausalMask(N, off, win)
        for i in range(N):
            for j in range(off + N):
                ok = (off + i) >= j and (win is None or (off + i) < j + win)
                assert m.arr[i, j] == ok
        assert m.causalEquivalent == (win is None)


def test_mask_mode_mapping():
    assert ops._mask_args(ops.Mask("")) == (0, 0)
    assert ops._mask_args(ops.Mask("causal")) == (1, 0)
    assert ops._mask_args(ops.createCausalMask(4, 8, None)) == (1, 0)
    assert ops._mask_args(ops.createCausalMask(4, 8, 6)) == (1, 6)
    # any other array mask is applied as given (mlxq_quantized_sdpa_array_mask)
    assert ops._mask_args(ops.Mask("array", np.ones((2, 2), bool))) == (ops._MASK_ARRAY, 0)
    with pytest.raises(ValueError):
        ops._mask_args(ops.Mask("bidir"))


def test_cache_make_mask_rules():
    """gemma4-base.ts:509-519 (QuantizedKVCache) and :1113-1123 (rotating)."""
    c = QuantizedKVCache(64, 4)
    assert c.makeMask(1, None).mode == ""
    assert c.makeMask(8, None).mode == "causal"
    c.offset = 10
    m = c.makeMask(8, None)
    assert m.mode == "array" and m.causalEquivalent and m.arr.shape == (8, 18)
    r = RotatingQuantizedKVCache(16, 64, 4)
    assert r.makeMask(1, None).mode == ""
    assert r.makeMask(4, None).mode == "causal"
    r.offset = 30
    m = r.makeMask(4, None)  # offset clamps to maxSize - 1 = 15; 15 + 4 > 16
    assert m.mode == "array" and m.window == 16 and m.arr.shape == (4, 19)


def test_gather_batch_maps():
    """gather_qmm's batch broadcast (x's leading dims against rhs_indices):
    SwitchGLU's expand_dims(x, (-2, -3)) against indices [B, L, k] makes
    output element (b, l, j) read x row (b, l) (src/model/gemma4.ts:434-438)."""
    from mlxq.ops import gather_batch_maps

    out, xm = gather_batch_maps((1, 2, 1), (1, 2, 2))  # tests/moe-ops.test.ts shapes
    assert out == (1, 2, 2) and xm.tolist() == [0, 0, 1, 1]
    out, xm = gather_batch_maps((4, 1, 1), (4, 1, 8))
    assert out == (4, 1, 8) and xm.tolist() == [i // 8 for i in range(32)]
    out, xm = gather_batch_maps((6,), (6,))  # sorted path: one x row per index
    assert out == (6,) and xm is None
    out, xm = gather_batch_maps((), (5,))  # one x broadcast to every index
    assert out == (5,) and xm.tolist() == [0] * 5
    out, xm = gather_batch_maps((3, 1), (1, 2))  # both sides broadcast
    assert out == (3, 2) and xm.tolist() == [0, 0, 1, 1, 2, 2]
