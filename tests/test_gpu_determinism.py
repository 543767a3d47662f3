"""GPU: every call that splits its reduction over workgroups is deterministic.

The reference's flash-decoding kernel merges its split-N partials in a fixed
order so repeated calls are bit-identical (src/model/fused-decode-kernel.ts:
14-18, :205-222).  The same holds here for each split path: the split-K
decode and its merge kernel (32k context, and the batched ring), the split
wide prefill, the tiled GEMM's split-K reduce and the sorted gather's work
list.  Each runs twice on the same inputs; the outputs must be equal bit for
bit.
"""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

BF16 = 12


def _random_triple(r, lead, D, gs, bits):
    """A quantized tensor with uniformly random codes and N(0, 0.1^2) bf16
    scales / biases (any bits are valid codes)."""
    from mlxq.array import DeviceArray, f32_to_bits
    from mlxq.ops import QuantizedTensor

    packed = r.integers(0, 2 ** 32, lead + (D * bits // 32,), dtype=np.uint64).astype(np.uint32)
    sb = [f32_to_bits(r.standard_normal(lead + (D // gs,)).astype(np.float32) * 0.1, BF16) for _ in range(2)]
    return QuantizedTensor(DeviceArray.fromNumpy(packed, 3), DeviceArray.fromNumpy(sb[0], BF16),
                           DeviceArray.fromNumpy(sb[1], BF16))


def _bf16(r, shape, scale=1.0):
    from mlxq.array import DeviceArray

    return DeviceArray.fromFloat32(r.standard_normal(shape).astype(np.float32) * scale, shape, BF16)


def _twice(fn):
    a = fn().rawNumpy()
    b = fn().rawNumpy()
    np.testing.assert_array_equal(a, b)
    return a


@pytest.mark.parametrize("case", ["decode_32k", "ring_b32_d256", "prefill_wide_split"])
def test_sdpa_split_paths_bit_identical(mlxq_dev, case):
    from mlxq import ops
    from mlxq.array import DeviceArray

    r = np.random.default_rng(11)
    vl = ro = None
    if case == "decode_32k":
        B, Hq, Hkv, L, D, N, scale, mask = 1, 32, 8, 1, 128, 32768, 128 ** -0.5, ops.Mask("")
    elif case == "ring_b32_d256":
        B, Hq, Hkv, L, D, N, scale, mask = 32, 16, 8, 1, 256, 4096, 1.0, ops.Mask("")
        vl = DeviceArray.fromNumpy(r.integers(512, 32769, B).astype(np.int32), 7)
        ro = DeviceArray.fromNumpy(r.integers(0, N, B).astype(np.int32), 7)
    else:
        B, Hq, Hkv, L, D, N, scale, mask = 1, 16, 2, 64, 512, 2048, 1.0, ops.Mask("causal")
    q = _bf16(r, (B, Hq, L, D))
    kq = _random_triple(r, (B, Hkv, N), D, 64, 4)
    vq = _random_triple(r, (B, Hkv, N), D, 64, 4)
    out = _twice(lambda: ops.quantizedSdpa(q, kq, vq, scale, mask, 64, 4, validLen=vl, ringOffset=ro))
    assert np.isfinite((out.astype(np.uint32) << 16).view(np.float32)).all()


@pytest.mark.parametrize("M,N,K", [(64, 14336, 4096), (16, 4096, 14336)])
def test_qmm_split_k_bit_identical(mlxq_dev, M, N, K):
    from mlxq import ops

    r = np.random.default_rng(M)
    x = _bf16(r, (M, K))
    w = _random_triple(r, (N,), K, 64, 4)
    _twice(lambda: ops.quantizedMatmul(x, w.packed, w.scales, w.biases, ops.QuantSpec(4, 64)))


def test_sorted_gather_bit_identical(mlxq_dev):
    from mlxq import ops
    from mlxq.array import DeviceArray

    r = np.random.default_rng(12)
    E, N, K, rows = 128, 1408, 2816, 4096
    w = _random_triple(r, (E, N), K, 64, 4)
    idx = DeviceArray.fromNumpy(np.sort(r.integers(0, E, rows)).astype(np.uint32), 3)
    x = _bf16(r, (rows, 1, K))
    _twice(lambda: ops.gatherQmm(x, w.packed, w.scales, w.biases, idx, ops.QuantSpec(4, 64), sortedIndices=True))
