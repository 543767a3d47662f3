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


@pytest.mark.parametrize("dtype,M,N,K", [
    (BF16, 1, 1000, 2048),   # ragged N
    (F16, 1, 333, 2816),     # 22 tiles (the tied-head and MoE gate_up K)
    (BF16, 1, 77, 14336),    # 112 tiles
    (F16, 1, 4097, 6144),    # one row past a workgroup multiple
    (BF16, 1, 9, 3072),      # fewer rows than one row tile
    (F16, 1, 50, 1280),      # 10 tiles
    (BF16, 2, 1000, 2048),   # two activation rows
    (F16, 2, 333, 2816),
    (BF16, 2, 4097, 14336),
])
def test_qmv_one_row_shapes(O, mlxq_dev, dtype, M, N, K):
    """One or two activation rows (qmv, 4-bit, group 64) against the float64
    reference: K from 10 to 112 tiles of 128 codes (a clamped duplicate tail
    at 22), ragged N, fewer rows than a row tile."""
    w = rng_t(O, (N, K), 13, dtype, 0.05)
    wq = O.quantize(w, 64, 4, dtype)
    x = rng_t(O, (M, K), 14, dtype)
    y = run_qmm(O, mlxq_dev, x, wq, 64, 4, dtype)
    assert_close(y, x.astype(np.float64) @ deq64(O, *wq, 64, 4, dtype).T, what="qmv", dtype=dtype)


@pytest.mark.parametrize("dtype,gs,M,N,K", [
    (BF16, 128, 12, 1000, 4096),  # 12 rows at group 128: a qmv plan with no compiled instance
    (F16, 128, 16, 15000, 512),   # the same at 16 rows, ragged N
    (BF16, 64, 1, 5000, 1024),
    (F16, 64, 4, 9000, 2048),
    (F16, 64, 2, 12345, 4096),    # odd N
    (BF16, 64, 1, 7001, 2048),    # 14 rows a workgroup (2 a CU on 256 CUs), a 1-row last one
    (F16, 64, 1, 13000, 1024),    # 13 rows a workgroup (4 a CU)
    (BF16, 64, 3, 15000, 1024),   # two row tiles, 30 rows a workgroup (2 a CU)
])
def test_qmm_small_m_shapes(O, mlxq_dev, dtype, gs, M, N, K):
    """Small-M shapes against float64, among them 9-16 activation rows at
    group 128 (one MFMA row block with 16-chunk x staging): the qmv plan for
    them has no compiled instance, and the call must go on to the tiled GEMM
    rather than fail; and plans whose workgroups do not come out a whole
    number a CU, which take 12-15 (one row tile) or 24-31 rows (two)."""
    w = rng_t(O, (N, K), 15, dtype, 0.05)
    wq = O.quantize(w, gs, 4, dtype)
    x = rng_t(O, (M, K), 16, dtype)
    y = run_qmm(O, mlxq_dev, x, wq, gs, 4, dtype)
    assert_close(y, x.astype(np.float64) @ deq64(O, *wq, gs, 4, dtype).T, what="small M", dtype=dtype)


@pytest.mark.parametrize("dtype,bits,gs,M,N,K", [
    (F16, 4, 64, 3, 200, 512),
    (F16, 8, 64, 5, 130, 768),
    (BF16, 8, 64, 17, 96, 1024),
    (BF16, 4, 128, 2, 77, 2048),
    (BF16, 8, 128, 33, 64, 256),
    (F16, 4, 128, 64, 50, 1280),
    # qmv with K not a whole number of 128-code tiles and / or a group count
    # that is not a multiple of 4 (scales staged one group at a time)
    (BF16, 4, 64, 1, 2816, 704),   # MoE down projection of the 26B-A4B model: 5.5 tiles, 11 groups
    (F16, 4, 64, 3, 100, 320),     # 2.5 tiles, 5 groups
    (BF16, 8, 64, 2, 90, 704),     # 8-bit: whole tiles, 11 groups
    (BF16, 4, 128, 1, 64, 640),    # group 128: 5 groups
    (F16, 4, 64, 16, 70, 448),     # two row blocks, 3.5 tiles, 7 groups
    # one wave for several output blocks (K of 2 tiles): each block stored
    (BF16, 4, 64, 16, 40, 256),    # 2 row blocks
    (F16, 4, 64, 12, 8192, 256),   # 2 row blocks x 2 row tiles
])
def test_qmm_mfma_variants(O, mlxq_dev, dtype, bits, gs, M, N, K):
    w = rng_t(O, (N, K), 3, dtype, 0.05)
    wq = O.quantize(w, gs, bits, dtype)
    x = rng_t(O, (M, K), 4, dtype)
    y = run_qmm(O, mlxq_dev, x, wq, gs, bits, dtype)
    assert_close(y, x.astype(np.float64) @ deq64(O, *wq, gs, bits, dtype).T, what="mfma variant", dtype=dtype)


@pytest.mark.parametrize("dtype,M,N,K", [
    (BF16, 64, 14336, 4096),   # up projection, no K split, rotated batches
    (BF16, 64, 4096, 14336),   # down projection, K split
    (F16, 17, 200, 1280),      # two row blocks, ragged N, a partial batch
    (BF16, 48, 96, 640),       # three row blocks, 5 K tiles (a partial batch)
    (F16, 32, 64, 1536),       # 12 K tiles: 3 batches, rotated
    (BF16, 33, 130, 2048),     # ragged M and N
    (BF16, 16, 4096, 14336),   # one row block (the M = 16 down projection)
])
def test_qmm_dma_kernel(O, mlxq_dev, dtype, M, N, K):
    """The direct-to-LDS pipelined kernel (4-bit, group 64, 16 < M <= 64 and
    the M <= 16 shapes qmv does not take) against the float64 reference:
    ragged M and N, partial and rotated batches, both dtypes."""
    w = rng_t(O, (N, K), 7, dtype, 0.05)
    wq = O.quantize(w, 64, 4, dtype)
    x = rng_t(O, (M, K), 8, dtype)
    y = run_qmm(O, mlxq_dev, x, wq, 64, 4, dtype)
    assert_close(y, x.astype(np.float64) @ deq64(O, *wq, 64, 4, dtype).T, what="dma", dtype=dtype)


def test_qmm_tile_at_dma_shapes(O, mlxq_dev, monkeypatch):
    """MLXQ_QMM_STREAM=0 keeps the tiled GEMM reachable at those shapes."""
    monkeypatch.setenv("MLXQ_QMM_STREAM", "0")
    w = rng_t(O, (256, 2048), 9, BF16, 0.05)
    wq = O.quantize(w, 64, 4, BF16)
    x = rng_t(O, (40, 2048), 10, BF16)
    y = run_qmm(O, mlxq_dev, x, wq, 64, 4, BF16)
    assert_close(y, x.astype(np.float64) @ deq64(O, *wq, 64, 4, BF16).T, what="tile", dtype=BF16)


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


# ---------------------------------------------------------------- gather_qmm

def _gather_ref(O, x, wq, idx_flat, x_map, gs, bits, dtype):
    """float64 per-expert reference: out[i] = x[x_map[i]] @ deq(W[idx[i]])^T."""
    p, s, b = wq
    M, K = x.shape[-2], x.shape[-1]
    xf = x.reshape(-1, M, K).astype(np.float64)
    out = []
    for i, e in enumerate(idx_flat):
        wd = deq64(O, p[e], s[e], b[e], gs, bits, dtype)
        out.append(xf[x_map[i]] @ wd.T)
    return np.stack(out)


def _gather(O, x, wq, idx, gs, bits, dtype, idx_dtype=3, sorted_indices=False):
    from mlxq import ops
    from mlxq.array import DeviceArray

    p, s, b = wq
    y = ops.gatherQmm(DeviceArray.fromFloat32(x, x.shape, dtype), DeviceArray.fromNumpy(p, 3),
                      DeviceArray.fromNumpy(s, dtype), DeviceArray.fromNumpy(b, dtype),
                      DeviceArray.fromNumpy(np.asarray(idx, np.uint32 if idx_dtype == 3 else np.int32), idx_dtype),
                      ops.QuantSpec(bits, gs), sorted_indices)
    return y.toFloat32()


@pytest.mark.parametrize("bits", [4, 8])
def test_gather_qmm_reference_case(O, mlxq_dev, bits):
    """tests/moe-ops.test.ts: 4 experts [16, 64] group 32 on the reference's LCG
    data (fp32), x [1, 2, 64] -> [1, 2, 1, 1, 64], indices [[2, 0], [1, 3]]:
    gather_qmm equals a per-expert quantized_matmul loop to < 1e-5 and the
    float64 oracle to the matmul bar."""
    from mlxq import ops
    from mlxq.array import DeviceArray

    E, OUT, IN, GS = 4, 16, 64, 32
    w = O.lcg_floats(E * OUT * IN, 7).reshape(E, OUT, IN)
    wq = O.quantize(w, GS, bits, F32)
    x = O.lcg_floats(2 * IN, 11).reshape(1, 2, IN)
    h = x.reshape(1, 2, 1, 1, IN)
    idx = np.array([2, 0, 1, 3], np.uint32).reshape(1, 2, 2)
    got = _gather(O, h, wq, idx, GS, bits, F32)
    assert got.shape == (1, 2, 2, 1, OUT)
    p, s, b = wq
    loop = np.zeros((2, 2, OUT), np.float32)
    for t in range(2):
        for j in range(2):
            e = int(idx[0, t, j])
            y = ops.quantizedMatmul(DeviceArray.fromFloat32(x[0, t:t + 1], (1, IN), F32), DeviceArray.fromNumpy(p[e], 3),
                                    DeviceArray.fromNumpy(s[e], F32), DeviceArray.fromNumpy(b[e], F32),
                                    ops.QuantSpec(bits, GS), True)
            loop[t, j] = y.toFloat32()[0]
    assert np.abs(got.reshape(2, 2, OUT) - loop).max() < 1e-5
    ref = _gather_ref(O, h, wq, idx.ravel(), [0, 0, 1, 1], GS, bits, F32)
    assert_close(got.reshape(4, 1, OUT), ref, what="gather ref case", dtype=F32)


@pytest.fixture(scope="module")
def experts_up(O):
    """16 experts of the 26B-A4B gate_up shape [1408, 2816], 4-bit group 64
    (docs/design/diffusion-gemma-port.md:357; 16 of the 128 experts)."""
    w = rng_t(O, (16, 1408, 2816), 31, BF16, 0.02)
    return O.quantize(w, 64, 4, BF16)


@pytest.mark.parametrize("B", [1, 4, 8])
def test_gather_qmm_moe_decode(O, mlxq_dev, experts_up, B):
    """SwitchGLU decode: x [B, 1, H] -> [B, 1, 1, 1, H] against top-8 indices
    [B, 1, 8] (qmv per (token, expert) through the row map)."""
    r = np.random.default_rng(40 + B)
    idx = np.stack([r.choice(16, 8, replace=False) for _ in range(B)]).astype(np.uint32).reshape(B, 1, 8)
    x = rng_t(O, (B, 1, 1, 1, 2816), 41 + B, BF16)
    got = _gather(O, x, experts_up, idx, 64, 4, BF16)
    assert got.shape == (B, 1, 8, 1, 1408)
    ref = _gather_ref(O, x, experts_up, idx.ravel(), [i // 8 for i in range(8 * B)], 64, 4, BF16)
    assert_close(got.reshape(8 * B, 1, 1408), ref, what=f"moe decode B={B}", dtype=BF16)


def test_gather_qmm_sorted_rows_and_bad_index(O, mlxq_dev, experts_up):
    """The sorted path (x [rows, 1, H], indices [rows] grouped by expert) and
    an expert index past the end (its row is zeros), int32 indices."""
    idx = np.array([0, 0, 3, 3, 3, 9, 15, 99], np.int32)
    x = rng_t(O, (8, 1, 2816), 50, BF16)
    got = _gather(O, x, experts_up, idx, 64, 4, BF16, idx_dtype=7)
    assert not got[7].any()
    ref = _gather_ref(O, x[:7], experts_up, idx[:7], list(range(7)), 64, 4, BF16)
    assert_close(got[:7], ref, what="sorted", dtype=BF16)


@pytest.mark.parametrize("path", ["dma", "tile"])
def test_gather_qmm_many_rows_per_expert(O, mlxq_dev, experts_up, monkeypatch, path):
    """M = 40 rows per gathered matmul through the batch map: the
    direct-to-LDS kernel, and (MLXQ_QMM_STREAM=0) the tiled GEMM."""
    if path == "tile":
        monkeypatch.setenv("MLXQ_QMM_STREAM", "0")
    idx = np.array([5, 2], np.uint32)
    x = rng_t(O, (2, 40, 2816), 51, BF16)
    got = _gather(O, x, experts_up, idx, 64, 4, BF16)
    ref = _gather_ref(O, x, experts_up, idx, [0, 1], 64, 4, BF16)
    assert_close(got, ref, what=f"{path} gather", dtype=BF16)


# ------------------------------------------------- gather_qmm, sorted rows

@pytest.fixture(scope="module")
def experts_small(O):
    """16 experts W [256, 512] ~ N(0, 0.02^2), 4-bit group 64, with their
    float64 dequantization."""
    w = rng_t(O, (16, 256, 512), 41, BF16, 0.02)
    wq = O.quantize(w, 64, 4, BF16)
    wd = np.stack([deq64(O, wq[0][e], wq[1][e], wq[2][e], 64, 4, BF16) for e in range(16)])
    return wq, wd


def _sorted_ref(x, wd, idx):
    """out[i] = x[i] @ deq(W[idx[i]])^T (an index past the experts: zeros)."""
    xf = x.reshape(len(idx), -1).astype(np.float64)
    out = np.zeros((len(idx), wd.shape[1]))
    for e in np.unique(idx):
        if 0 <= e < len(wd):
            rows = np.nonzero(idx == e)[0]
            out[rows] = xf[rows] @ wd[e].T
    return out.reshape(len(idx), 1, -1)


@pytest.mark.parametrize("rows,order", [(512, "sorted"), (2048, "sorted"), (512, "unsorted"), (300, "one expert")])
def test_gather_qmm_sorted_grouped_gemm(O, mlxq_dev, experts_small, rows, order):
    """SwitchGLU's sorted call (src/model/gemma4.ts:441-473): x [rows, 1, K]
    in expert order, indices [rows], sortedIndices=True -> expert runs as GEMM
    blocks (32-row blocks at 512 rows over 16 experts, 64-row blocks at 2048,
    runs longer than a block).  Unsorted indices with the flag set and a
    single expert's run give the same results; equal to the per-row gather."""
    wq, wd = experts_small
    r = np.random.default_rng(rows)
    if order == "one expert":
        idx = np.full(rows, 7, np.uint32)
    else:
        idx = r.integers(0, 16, rows).astype(np.uint32)
        if order == "sorted":
            idx.sort()
    x = rng_t(O, (rows, 1, 512), 60 + rows, BF16)
    got = _gather(O, x, wq, idx, 64, 4, BF16, sorted_indices=True)
    assert_close(got, _sorted_ref(x, wd, idx), what=f"sorted gather {rows} {order}", dtype=BF16)
    per_row = _gather(O, x, wq, idx, 64, 4, BF16)
    assert_close(got, per_row, atol=1e-2, rtol=1e-3, what="sorted vs per-row", dtype=BF16)


def test_gather_qmm_sorted_bad_index_and_repeat(O, mlxq_dev, experts_small):
    """Sorted rows whose last run indexes past the experts give zero rows, and
    a second, smaller call through the same workspace is still exact."""
    wq, wd = experts_small
    idx = np.sort(np.random.default_rng(5).integers(0, 16, 640)).astype(np.uint32)
    idx[-40:] = 99
    x = rng_t(O, (640, 1, 512), 77, BF16)
    got = _gather(O, x, wq, idx, 64, 4, BF16, sorted_indices=True)
    assert not got[-40:].any()
    assert_close(got, _sorted_ref(x, wd, idx), what="sorted bad index", dtype=BF16)
    idx2 = np.sort(np.random.default_rng(6).integers(0, 16, 96)).astype(np.uint32)
    x2 = rng_t(O, (96, 1, 512), 78, BF16)
    got2 = _gather(O, x2, wq, idx2, 64, 4, BF16, sorted_indices=True)
    assert_close(got2, _sorted_ref(x2, wd, idx2), what="sorted second call", dtype=BF16)


@pytest.fixture(scope="module")
def experts_many(O):
    """512 experts W [128, 256] ~ N(0, 0.02^2), 4-bit group 64, with their
    float64 dequantization (few rows an expert: 32-row GEMM blocks)."""
    w = rng_t(O, (512, 128, 256), 43, BF16, 0.02)
    wq = O.quantize(w, 64, 4, BF16)
    wd = deq64(O, wq[0], wq[1], wq[2], 64, 4, BF16)
    return wq, wd


@pytest.mark.parametrize("rows,experts", [(16384, "few"), (16384, "many"), (20000, "few"), (20000, "many"),
                                          (4106, "few"), (4106, "many")])
def test_gather_qmm_sorted_past_one_index_stage(O, mlxq_dev, experts_small, experts_many, rows, experts):
    """The segments kernel builds the work list 4096 rows a pass: 16384 rows
    (the reference's 2048-token prefill chunk x top-8) end exactly on a pass
    boundary, 20000 rows have one expert's run straddling row 16384 (its run
    start and open item carried into the next pass), and 4106 rows end in a
    10-row pass inside a run that starts no block there (a pass with no item
    of its own).  16 experts give 64-row blocks, 512 experts 32-row blocks.
    Against the fp64 reference and the per-row gather."""
    wq, wd = experts_small if experts == "few" else experts_many
    E, K = wd.shape[0], wd.shape[2]
    r = np.random.default_rng(rows + E)
    idx = np.sort(r.integers(0, E, rows)).astype(np.uint32)
    if rows == 20000:
        idx[16360:16410] = idx[16360]  # one run across the pass boundary (order kept)
        assert idx[16383] == idx[16384]
    if rows == 4106:
        idx[-30:] = E - 1  # one run from row 4076: its next block would start at 4108
        idx[:-30] = np.minimum(idx[:-30], E - 2)
        idx.sort()
    x = rng_t(O, (rows, 1, K), 90 + rows, BF16)
    got = _gather(O, x, wq, idx, 64, 4, BF16, sorted_indices=True)
    assert_close(got, _sorted_ref(x, wd, idx), what=f"sorted gather {rows} rows, {E} experts", dtype=BF16)
    per_row = _gather(O, x, wq, idx, 64, 4, BF16)
    assert_close(got, per_row, what="sorted vs per-row", dtype=BF16)
