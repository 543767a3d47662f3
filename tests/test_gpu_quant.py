"""GPU: quantize / dequantize / kv_append bit-exact against the oracle."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

BF16, F16, F32 = 12, 9, 10


def rng_t(O, shape, seed, dtype, scale=1.0):
    r = np.random.default_rng(seed)
    return O.round_t(r.standard_normal(shape).astype(np.float32) * scale, dtype)


def upload(mlxq_dev, x, dtype):
    return mlxq_dev.DeviceArray.fromFloat32(x, x.shape, dtype)


@pytest.mark.parametrize("dtype", [BF16, F16, F32])
@pytest.mark.parametrize("bits,gs", [(2, 32), (2, 64), (4, 32), (4, 64), (4, 128), (8, 32), (8, 64), (8, 128)])
def test_quantize_bit_exact(O, mlxq_dev, dtype, bits, gs):
    from mlxq import ops

    w = rng_t(O, (67, 384), 100 + bits + gs, dtype, 3.0)
    w[3, :gs] = 0.0                           # all-zero group: scale 1e-7 path
    w[5, :gs] = np.float32(-1.5)              # constant negative group
    w[7, gs:2 * gs] = np.linspace(-2, 2, gs)  # exact ties
    w = O.round_t(w, dtype)
    qt = ops.quantize(upload(mlxq_dev, w, dtype), gs, bits)
    p, s, b = O.quantize(w, gs, bits, dtype)
    np.testing.assert_array_equal(qt.packed.rawNumpy(), p)
    np.testing.assert_array_equal(qt.scales.rawNumpy(), s)
    np.testing.assert_array_equal(qt.biases.rawNumpy(), b)


def test_quantize_bit_exact_32k_cache(O, mlxq_dev):
    """The decode cache of the 32k-context workload: K [1, 8, 32768, 128] bf16, 4-bit."""
    from mlxq import ops

    k = rng_t(O, (1, 8, 32768, 128), 7, BF16)
    qt = ops.quantize(upload(mlxq_dev, k, BF16), 64, 4)
    p, s, b = O.quantize(k, 64, 4, BF16)
    np.testing.assert_array_equal(qt.packed.rawNumpy(), p)
    np.testing.assert_array_equal(qt.scales.rawNumpy(), s)
    np.testing.assert_array_equal(qt.biases.rawNumpy(), b)


@pytest.mark.parametrize("dtype", [BF16, F16, F32])
@pytest.mark.parametrize("bits,gs", [(2, 64), (4, 64), (8, 32), (8, 128)])
def test_dequantize_bit_exact(O, mlxq_dev, dtype, bits, gs):
    from mlxq import ops

    w = rng_t(O, (33, 256), 5, dtype)
    p, s, b = O.quantize(w, gs, bits, dtype)
    d = ops.dequantize(mlxq_dev.DeviceArray.fromNumpy(p, 3), mlxq_dev.DeviceArray.fromNumpy(s, dtype),
                       mlxq_dev.DeviceArray.fromNumpy(b, dtype), ops.QuantSpec(bits, gs))
    np.testing.assert_array_equal(d.toFloat32(), O.dequantize(p, s, b, gs, bits, dtype))


def test_kv_append_wraps_the_ring(O, mlxq_dev):
    """Rows land at (write_pos + r) mod capacity of every head."""
    from mlxq import _lib
    from mlxq.array import DeviceArray, Dtype

    heads, cap, S, D, gs, bits = 6, 40, 7, 128, 64, 4
    x = rng_t(O, (heads, S, D), 9, BF16)
    pk = DeviceArray.zeros((heads, cap, D * bits // 32), Dtype.uint32)
    sc = DeviceArray.zeros((heads, cap, D // gs), BF16)
    bi = DeviceArray.zeros((heads, cap, D // gs), BF16)
    _lib.call("mlxq_kv_append", upload(mlxq_dev, x, BF16).ptr, BF16, heads, S, D, gs, bits, pk.ptr, sc.ptr, bi.ptr,
              cap, 37, None)
    p, s, b = O.quantize(x, gs, bits, BF16)
    slots = [(37 + r) % cap for r in range(S)]
    got_p, got_s = pk.rawNumpy(), sc.rawNumpy()
    np.testing.assert_array_equal(got_p[:, slots], p)
    np.testing.assert_array_equal(got_s[:, slots], s)
    np.testing.assert_array_equal(bi.rawNumpy()[:, slots], b)
    untouched = [i for i in range(cap) if i not in slots]
    assert not got_p[:, untouched].any() and not got_s[:, untouched].any()


@pytest.mark.parametrize("dtype,bits,gs", [(BF16, 4, 64), (F16, 8, 32), (BF16, 8, 128), (F16, 4, 128), (F32, 2, 64)])
@pytest.mark.parametrize("id_dtype", [3, 7])
def test_embedding_encode_bit_exact(O, mlxq_dev, dtype, bits, gs, id_dtype):
    """QuantizedEmbedding.encode (take rows of packed / scales / biases, then
    dequantize): bit-exact against the oracle's dequantize of the gathered
    rows, ids [1, L] in int32 or uint32, repeated ids, an id past the
    vocabulary (zero row; for int32 also a negative id)."""
    from mlxq import ops
    from mlxq.layers import QuantizedEmbedding

    vocab, D = 1000, 256
    w = rng_t(O, (vocab, D), 60 + bits, dtype)
    p, s, b = O.quantize(w, gs, bits, dtype)
    ids = np.array([[0, 999, 17, 17, 512, 1000, 3, 998]], np.int64)
    if id_dtype == 7:
        ids[0, 6] = -5
    emb = QuantizedEmbedding(mlxq_dev.DeviceArray.fromNumpy(p, 3), mlxq_dev.DeviceArray.fromNumpy(s, dtype),
                             mlxq_dev.DeviceArray.fromNumpy(b, dtype), ops.QuantSpec(bits, gs))
    dev_ids = mlxq_dev.DeviceArray.fromNumpy(ids.astype(np.uint32 if id_dtype == 3 else np.int32), id_dtype)
    got = emb.encode(dev_ids).toFloat32()
    assert got.shape == (1, 8, D)
    full = O.dequantize(p, s, b, gs, bits, dtype)
    for j, i in enumerate(ids[0]):
        if 0 <= i < vocab:
            np.testing.assert_array_equal(got[0, j], full[i])
        else:
            assert not got[0, j].any()


def test_embedding_tied_head(O, mlxq_dev):
    """QuantizedEmbedding.asLinear: h [1, 3, 2816] against a 16384-row slice of
    the 26B-A4B embedding table (4-bit group 64), fp32-accumulated logits."""
    from conftest import assert_close
    from mlxq import ops
    from mlxq.layers import QuantizedEmbedding

    vocab, H = 16384, 2816
    w = rng_t(O, (vocab, H), 70, BF16, 0.02)
    p, s, b = O.quantize(w, 64, 4, BF16)
    emb = QuantizedEmbedding(mlxq_dev.DeviceArray.fromNumpy(p, 3), mlxq_dev.DeviceArray.fromNumpy(s, BF16),
                             mlxq_dev.DeviceArray.fromNumpy(b, BF16), ops.QuantSpec(4, 64))
    h = rng_t(O, (1, 3, H), 71, BF16)
    got = emb.asLinear(upload(mlxq_dev, h, BF16)).toFloat32()
    # fp64 reference on unrounded dequantized weights (quantized_matmul never
    # rounds s*c + b to T)
    p64 = O.unpack_codes(p, 4).astype(np.float64)
    wd = O.from_t(s, BF16).astype(np.float64).repeat(64, -1) * p64 + O.from_t(b, BF16).astype(np.float64).repeat(64, -1)
    ref = h.astype(np.float64).reshape(3, H) @ wd.T
    assert_close(got.reshape(3, vocab), ref, what="tied head", dtype=BF16)
