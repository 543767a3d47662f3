"""GPU: quantized_matmul against the fp32 reference (float64 numpy on the
oracle-dequantized weights).  Tolerance (matmul outputs, fp32 accumulation):
|y - ref| <= 1e-2 + 1e-3 |ref| + half an ulp of the output dtype."""
import numpy as np
import pytest

from conftest import assert_close

pytestmark = pytest.mark.gpu

BF16, F16, F32 = 12, 9, 10


def rng_t(O, shape, seed, dtype, scale=1.0):
    r = np.random.default_rng(seed)
    return O.round_t(r.standard_normal(shape).astype(np.float32) * scale, dtype)


def deq64(O, p, s, b, gs, bits, dtype):
    c = O.unpack_codes(p, bits).astype(np.float64)
    return O.from_t(s, dtype).astype(np.float64).repeat(gs, -1) * c + O.from_t(b, dtype).astype(np.float64).repeat(gs, -1)


def run_qmm(O, mlxq_dev, x, wq, gs, bits, dtype, transpose=True):
    from mlxq import ops
    from mlxq.array import DeviceArray

    p, s, b = wq
    y = ops.quantizedMatmul(DeviceArray.fromFloat32(x, x.shape, dtype), DeviceArray.fromNumpy(p, 3),
                            DeviceArray.fromNumpy(s, dtype), DeviceArray.fromNumpy(b, dtype),
                            ops.QuantSpec(bits, gs), transpose)
    return y.toFloat32()


@pytest.fixture(scope="module")
def w_up(O):
    """W [14336, 4096] ~ N(0, 0.02^2), 4-bit group 64 (the MLP up/gate shape)."""
    w = rng_t(O, (14336, 4096), 1, BF16, 0.02)
    wq = O.quantize(w, 64, 4, BF16)
    return wq, deq64(O, *wq, 64, 4, BF16)


@pytest.fixture(scope="module")
def w_down(O):
    w = rng_t(O, (4096, 14336), 2, BF16, 0.02)
    wq = O.quantize(w, 64, 4, BF16)
    return wq, deq64(O, *wq, 64, 4, BF16)


@pytest.mark.parametrize("M", [1, 4, 16, 64])
def test_qmv_qmm_up_proj(O, mlxq_dev, w_up, M):
    wq, wd = w_up
    x = rng_t(O, (M, 4096), 10 + M, BF16)
    y = run_qmm(O, mlxq_dev, x, wq, 64, 4, BF16)
    assert_close(y, x.astype(np.float64) @ wd.T, what=f"up M={M}", dtype=BF16)


@pytest.mark.parametrize("M", [1, 4, 16, 64])
def test_qmv_qmm_down_proj(O, mlxq_dev, w_down, M):
    wq, wd = w_down
    x = rng_t(O, (M, 14336), 20 + M, BF16)
    y = run_qmm(O, mlxq_dev, x, wq, 64, 4, BF16)
    assert_close(y, x.astype(np.float64) @ wd.T, what=f"down M={M}", dtype=BF16)


@pytest.mark.parametrize("dtype,bits,gs,M,N,K", [
    (F16, 4, 64, 3, 200, 512),
    (F16, 8, 64, 5, 130, 768),
    (BF16, 8, 64, 17, 96, 1024),
    (BF16, 4, 128, 2, 77, 2048),
    (BF16, 8, 128, 33, 64, 256),
    (F16, 4, 128, 64, 50, 1280),
])
def test_qmm_mfma_variants(O, mlxq_dev, dtype, bits, gs, M, N, K):
    w = rng_t(O, (N, K), 3, dtype, 0.05)
    wq = O.quantize(w, gs, bits, dtype)
    x = rng_t(O, (M, K), 4, dtype)
    y = run_qmm(O, mlxq_dev, x, wq, gs, bits, dtype)
    assert_close(y, x.astype(np.float64) @ deq64(O, *wq, gs, bits, dtype).T, what="mfma variant", dtype=dtype)


@pytest.mark.parametrize("dtype,bits,gs,transpose", [
    (BF16, 4, 64, False), (F16, 8, 32, False), (BF16, 2, 64, True), (F32, 4, 64, True), (BF16, 4, 32, True)])
def test_qmm_generic_paths(O, mlxq_dev, dtype, bits, gs, transpose):
    M, K, N = 4, 256, 192
    w = rng_t(O, (N, K) if transpose else (K, N), 5, dtype, 0.05)
    wq = O.quantize(w, gs, bits, dtype)
    x = rng_t(O, (M, K), 6, dtype)
    y = run_qmm(O, mlxq_dev, x, wq, gs, bits, dtype, transpose)
    wd = deq64(O, *wq, gs, bits, dtype)
    assert_close(y, x.astype(np.float64) @ (wd.T if transpose else wd), what="generic", dtype=dtype)


def test_qmm_batched_broadcast(O, mlxq_dev):
    """x [2, 4, 3, 128] against w [2, 1, 40, .] broadcast over axis 1 (the
    expand_dims(-3) GQA pattern of quantizedSdpaUnfused)."""
    from mlxq import ops
    from mlxq.array import DeviceArray

    gs, bits = 64, 4
    x = rng_t(O, (2, 4, 3, 128), 7, BF16)
    w = rng_t(O, (2, 1, 40, 128), 8, BF16)
    p, s, b = O.quantize(w, gs, bits, BF16)
    y = ops.quantizedMatmul(DeviceArray.fromFloat32(x, x.shape, BF16), DeviceArray.fromNumpy(p, 3),
                            DeviceArray.fromNumpy(s, BF16), DeviceArray.fromNumpy(b, BF16), ops.QuantSpec(bits, gs))
    ref = O.qmm(x.reshape(8, 3, 128), p.reshape(2, 40, 16), s.reshape(2, 40, 2), b.reshape(2, 40, 2), gs, bits, BF16)
    assert_close(y.toFloat32().reshape(8, 3, 40), ref, what="batched", dtype=BF16)


@pytest.mark.parametrize("dtype,bits,gs,lead,M,N,K", [
    (BF16, 4, 32, (), 24, 300, 4096),     # 32 x 128 tiles, K split 8 ways
    (F16, 8, 128, (), 40, 264, 2048),     # 64 x 64 tiles, a K-step is half a group
    (BF16, 8, 64, (), 130, 512, 1024),    # ragged M tiles
    (F16, 4, 64, (), 20, 77, 8192),       # N % 4 != 0: one split over a long K
    (BF16, 4, 64, (3,), 33, 96, 2048),    # batch 3 against one broadcast w, split K
    (BF16, 4, 128, (), 512, 8192, 512),   # 128 x 128 tiles
    (F16, 8, 32, (), 100, 136, 3072),     # two group parts per K-step, split K
])
def test_qmm_tile(O, mlxq_dev, dtype, bits, gs, lead, M, N, K):
    """The tiled MFMA GEMM (M beyond qmv, or K too long for qmv's x slices):
    every bits / group_size / dtype pairing, split-K partials and the
    reduce, tiles cut by M and N."""
    w = rng_t(O, (N, K), 11, dtype, 0.05)
    wq = O.quantize(w, gs, bits, dtype)
    x = rng_t(O, lead + (M, K), 12, dtype)
    y = run_qmm(O, mlxq_dev, x, wq, gs, bits, dtype)
    assert_close(y, x.astype(np.float64) @ deq64(O, *wq, gs, bits, dtype).T, what="tile", dtype=dtype)
