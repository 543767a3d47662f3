"""GPU: quantized SDPA against the oracle.

Bar: |out - fp32 ref| <= 1e-2 + 1e-3 |ref| + half an ulp of T, elementwise
(fp32 accumulation throughout; the output itself is rounded to T).  On the
reference's own test data, the difference to its rounding-point restatement
(quantizedSdpaUnfused in T) must also stay under 0.02, the bound
tests/fused-decode-kernel.test.ts:61 holds the reference's fused kernel to.
"""
import numpy as np
import pytest

from conftest import assert_close

pytestmark = pytest.mark.gpu

BF16, F16, F32 = 12, 9, 10


def rng_t(O, shape, seed, dtype, scale=1.0):
    r = np.random.default_rng(seed)
    return O.round_t(r.standard_normal(shape).astype(np.float32) * scale, dtype)


def upload_triple(mlxq_dev, t, dtype):
    from mlxq.array import DeviceArray
    from mlxq.ops import QuantizedTensor

    return QuantizedTensor(DeviceArray.fromNumpy(t[0], 3), DeviceArray.fromNumpy(t[1], dtype),
                           DeviceArray.fromNumpy(t[2], dtype))


def run(O, mlxq_dev, q, kq, vq, dtype, scale, gs, bits, mask=None, valid=None, ring=None):
    from mlxq import ops
    from mlxq.array import DeviceArray

    dq = DeviceArray.fromFloat32(q, q.shape, dtype)
    vl = DeviceArray.fromNumpy(np.asarray(valid, np.int32), 7) if valid is not None else None
    ro = DeviceArray.fromNumpy(np.asarray(ring, np.int32), 7) if ring is not None else None
    out = ops.quantizedSdpa(dq, upload_triple(mlxq_dev, kq, dtype), upload_triple(mlxq_dev, vq, dtype), scale,
                            mask or ops.Mask(""), gs, bits, validLen=vl, ringOffset=ro)
    return out.toFloat32()


def case(O, B, Hq, Hkv, L, N, D, gs, bits, dtype, seed):
    q = rng_t(O, (B, Hq, L, D), seed, dtype)
    kq = O.quantize(rng_t(O, (B, Hkv, N, D), seed + 1, dtype), gs, bits, dtype)
    vq = O.quantize(rng_t(O, (B, Hkv, N, D), seed + 2, dtype), gs, bits, dtype)
    return q, kq, vq


def check(O, got, q, kq, vq, dtype, scale, gs, bits, tag, **geo):
    ref = O.sdpa(q, kq, vq, scale=scale, gs=gs, bits=bits, dtype=dtype, **geo)
    assert_close(got, ref, what=tag, dtype=dtype)


def test_decode_8bit_fp16_1k(O, mlxq_dev):
    """B=1, Hq=16, Hkv=4, D=128, N=1024, fp16, 8-bit group 64, scale 1/sqrt(128)."""
    q, kq, vq = case(O, 1, 16, 4, 1, 1024, 128, 64, 8, F16, 0)
    s = 1 / np.sqrt(128)
    check(O, run(O, mlxq_dev, q, kq, vq, F16, s, 64, 8), q, kq, vq, F16, s, 64, 8, "c1")


def test_decode_4bit_bf16_32k(O, mlxq_dev):
    """B=1, Hq=32, Hkv=8, D=128, N=32768, bf16, 4-bit group 64."""
    q, kq, vq = case(O, 1, 32, 8, 1, 32768, 128, 64, 4, BF16, 1)
    s = 1 / np.sqrt(128)
    check(O, run(O, mlxq_dev, q, kq, vq, BF16, s, 64, 4), q, kq, vq, BF16, s, 64, 4, "c2")


def test_decode_batched_ring_window(O, mlxq_dev):
    """B=32, Hq=16, Hkv=8, D=256, window 4096, per-row lengths in [512, 32768]
    (attended: min(len, 4096)) and ring write offsets in [0, 4096)."""
    r = np.random.default_rng(3)
    B, W = 32, 4096
    lens = r.integers(512, 32769, B).astype(np.int32)
    lens[:3] = [512, 4095, 4096]
    ring = r.integers(0, W, B).astype(np.int32)
    q, kq, vq = case(O, B, 16, 8, 1, W, 256, 64, 4, BF16, 4)
    got = run(O, mlxq_dev, q, kq, vq, BF16, 1.0, 64, 4, valid=lens, ring=ring)
    check(O, got, q, kq, vq, BF16, 1.0, 64, 4, "c3", valid_len=lens, ring_off=ring)


@pytest.mark.parametrize("gs,dtype", [(32, F16), (128, BF16)])
def test_decode_ring_four_wave_workgroups(O, mlxq_dev, gs, dtype):
    """Rotating rows on the 4-wave decode workgroups (4-bit D 256, 16 rows x
    8 kv heads x 9 chunks of a 8192-slot ring: two or more workgroups a CU
    on a 256-CU part) at group sizes 32 and 128: short rows, full rings cut
    at physical slots, and wrapped windows."""
    r = np.random.default_rng(gs)
    B, W = 16, 8192
    lens = r.integers(100, 20000, B).astype(np.int32)
    lens[:4] = [1, 8191, 8192, 8193]
    ring = r.integers(0, W, B).astype(np.int32)
    q, kq, vq = case(O, B, 16, 8, 1, W, 256, gs, 4, dtype, 60 + gs)
    got = run(O, mlxq_dev, q, kq, vq, dtype, 0.0625, gs, 4, valid=lens, ring=ring)
    check(O, got, q, kq, vq, dtype, 0.0625, gs, 4, f"ring gs{gs}", valid_len=lens, ring_off=ring)


@pytest.mark.parametrize("Hq,Hkv,D", [(32, 8, 128), (16, 8, 256)])
def test_decode_32k_scale_one(O, mlxq_dev, Hq, Hkv, D):
    """Gemma4 calls quantizedSdpa with scale 1 (src/model/gemma4-base.ts:1282-1285):
    unit-normal q and k then give scores with a spread of sqrt(D), the most
    peaked softmax the decode kernels see.  The 32k-context shape (nRep 4,
    D 128) and the D 256 / nRep 2 shape at 32k, 4-bit group 64, bf16."""
    q, kq, vq = case(O, 1, Hq, Hkv, 1, 32768, D, 64, 4, BF16, 21 + D)
    check(O, run(O, mlxq_dev, q, kq, vq, BF16, 1.0, 64, 4), q, kq, vq, BF16, 1.0, 64, 4, f"32k scale 1 D{D}")


@pytest.mark.parametrize("B,Hq,Hkv,N,D,gs,bits,dtype", [
    (1, 4, 2, 333, 256, 64, 4, BF16),     # fused-decode-kernel.test.ts site shapes, N=333
    (1, 4, 2, 333, 256, 64, 8, BF16),
    (2, 8, 8, 77, 128, 32, 4, BF16),      # no GQA, group 32, short
    (1, 16, 2, 1000, 128, 128, 8, F16),   # nRep 8, group 128
    (3, 6, 3, 129, 128, 64, 4, F16),      # nRep 2, odd sizes
    (1, 4, 1, 4100, 64, 32, 8, BF16),     # D=64
    (1, 2, 2, 1, 128, 64, 4, BF16),       # one key
    (1, 8, 2, 65537, 128, 64, 4, BF16),   # many chunks, ragged tail
])
def test_decode_shapes(O, mlxq_dev, B, Hq, Hkv, N, D, gs, bits, dtype):
    q, kq, vq = case(O, B, Hq, Hkv, 1, N, D, gs, bits, dtype, N)
    check(O, run(O, mlxq_dev, q, kq, vq, dtype, 0.125, gs, bits), q, kq, vq, dtype, 0.125, gs, bits, "shape")


@pytest.mark.parametrize("B,Hq,Hkv,N,D,gs,bits,dtype", [
    (1, 32, 1, 150, 128, 64, 4, BF16),    # nRep 32: past the MFMA kernels' 16 head rows
    (1, 4, 2, 200, 128, 64, 2, BF16),     # 2-bit
    (1, 4, 2, 150, 128, 64, 4, F32),      # fp32 activations
])
def test_decode_generic_shapes(O, mlxq_dev, B, Hq, Hkv, N, D, gs, bits, dtype):
    q, kq, vq = case(O, B, Hq, Hkv, 1, N, D, gs, bits, dtype, 9)
    check(O, run(O, mlxq_dev, q, kq, vq, dtype, 1.0, gs, bits), q, kq, vq, dtype, 1.0, gs, bits, "generic")


@pytest.mark.parametrize("B,Hq,Hkv,N,D,gs,bits,dtype,scale", [
    (1, 16, 2, 4096, 512, 64, 4, BF16, 1.0),    # Gemma4 full attention (src/config.ts:150-156): nRep 8, D 512
    (1, 16, 1, 333, 512, 64, 4, BF16, 1.0),     # the 12B full-attention site: nRep 16
    (2, 16, 2, 1000, 512, 128, 8, F16, 1.0),    # group 128, 8-bit
    (1, 16, 2, 777, 256, 32, 4, BF16, 0.0625),  # nRep 8 x 8 groups at D 256
    (1, 32, 2, 3000, 128, 64, 8, BF16, 0.125),  # nRep 16 at D 128
    (1, 8, 1, 100, 512, 64, 4, F16, 1.0),       # one chunk: outputs written by the kernel itself
    (1, 16, 2, 33001, 512, 64, 4, BF16, 1.0),   # 32k context, ragged last tile
])
def test_decode_wide(O, mlxq_dev, B, Hq, Hkv, N, D, gs, bits, dtype, scale):
    """Decode with more (head, group) score columns than one 16-wide MFMA
    tile holds: the wide kernel (heads as MFMA rows, exact K operands, V
    dequantized through LDS) against the fp64 oracle."""
    q, kq, vq = case(O, B, Hq, Hkv, 1, N, D, gs, bits, dtype, N + 1)
    check(O, run(O, mlxq_dev, q, kq, vq, dtype, scale, gs, bits), q, kq, vq, dtype, scale, gs, bits, "wide")


@pytest.mark.parametrize("gs,dtype", [(64, F16), (32, BF16), (128, BF16)])
def test_decode_d256_four_wave_workgroups(O, mlxq_dev, gs, dtype):
    """4-bit D 256 with 512 key chunks in the launch (8 rows x 8 kv heads x
    8 chunks of 1024 keys): two or more workgroups a CU on a 256-CU part, so
    the launcher takes 4-wave workgroups with 8 tiles a wave.  Scale 1 (the
    most peaked softmax), every group size."""
    q, kq, vq = case(O, 8, 16, 8, 1, 8192, 256, gs, 4, dtype, 40 + gs)
    check(O, run(O, mlxq_dev, q, kq, vq, dtype, 1.0, gs, 4), q, kq, vq, dtype, 1.0, gs, 4, f"d256 gs{gs}")


def test_decode_wide_ring(O, mlxq_dev):
    """Rotating rows at the Gemma4 full-attention shape: per-row valid lengths
    (short, one short of the ring, full, wrapped past it) and ring offsets."""
    B, W = 4, 2048
    lens = np.array([100, 2047, 2048, 5000], np.int32)
    ring = np.random.default_rng(8).integers(0, W, B).astype(np.int32)
    q, kq, vq = case(O, B, 16, 2, 1, W, 512, 64, 4, BF16, 21)
    got = run(O, mlxq_dev, q, kq, vq, BF16, 1.0, 64, 4, valid=lens, ring=ring)
    check(O, got, q, kq, vq, BF16, 1.0, 64, 4, "wide ring", valid_len=lens, ring_off=ring)


@pytest.mark.parametrize("B,Hq,Hkv,L,N,D,gs,bits,dtype,scale,window", [
    (1, 16, 2, 70, 600, 512, 64, 4, BF16, 1.0, 0),      # Gemma4 full attention: nRep 8, D 512, scale 1
    (1, 16, 2, 33, 300, 512, 128, 8, F16, 1.0, 0),      # group 128, 8-bit
    (2, 8, 2, 40, 257, 256, 32, 4, BF16, 0.0625, 0),    # D 256, 8 groups, batch 2
    (1, 4, 4, 129, 129, 256, 64, 8, BF16, 0.0625, 50),  # prompt (queries = keys) under a window
    (1, 8, 1, 17, 2000, 512, 64, 4, BF16, 1.0, 0),      # short chunk over a long cache (keys split 7 ways)
    (1, 16, 2, 24, 4096, 512, 64, 4, BF16, 1.0, 1000),  # 16 key splits under a window: empty and fully masked splits
    (2, 8, 1, 9, 3000, 256, 32, 8, F16, 0.0625, 0),     # batch 2, 11 key splits
])
def test_prefill_wide(O, mlxq_dev, B, Hq, Hkv, L, N, D, gs, bits, dtype, scale, window):
    """Chunked prefill at head_dim 256 / 512 (the wide MFMA kernel: 16 rows
    per wave, exact K operands, V dequantized through LDS), bottom-right
    causal (+ window), against the fp64 oracle."""
    from mlxq import ops

    q, kq, vq = case(O, B, Hq, Hkv, L, N, D, gs, bits, dtype, 30 + L)
    got = run(O, mlxq_dev, q, kq, vq, dtype, scale, gs, bits, mask=ops.createCausalMask(L, N - L, window or None))
    check(O, got, q, kq, vq, dtype, scale, gs, bits, "prefill wide", causal=True, window=window)


def test_decode_empty_rows_are_zero(O, mlxq_dev):
    q, kq, vq = case(O, 3, 8, 2, 1, 64, 128, 64, 4, BF16, 5)
    got = run(O, mlxq_dev, q, kq, vq, BF16, 1.0, 64, 4, valid=[0, 10, 0], ring=[3, 7, 0])
    assert not got[0].any() and not got[2].any()
    check(O, got[1:2], q[1:2], tuple(a[1:2] for a in kq), tuple(a[1:2] for a in vq), BF16, 1.0, 64, 4, "empty",
          valid_len=np.array([10], np.int32), ring_off=np.array([7], np.int32))


@pytest.mark.parametrize("L,N,window", [(16, 300, 0), (7, 50, 13), (64, 1217, 0), (33, 700, 100)])
def test_prefill_causal(O, mlxq_dev, L, N, window):
    from mlxq import ops

    q, kq, vq = case(O, 1, 8, 2, L, N, 128, 64, 4, BF16, 11)
    mask = ops.createCausalMask(L, N - L, window or None)
    got = run(O, mlxq_dev, q, kq, vq, BF16, 0.125, 64, 4, mask=mask)
    check(O, got, q, kq, vq, BF16, 0.125, 64, 4, "prefill", causal=True, window=window)


@pytest.mark.parametrize("KV,nRep,L,N,D,gs,bits", [  # tests/fused-sdpa.test.ts:66-72
    (2, 4, 96, 448, 64, 64, 8), (2, 4, 96, 1217, 64, 64, 8), (2, 4, 96, 1217, 64, 64, 4),
    (4, 1, 64, 700, 64, 32, 8), (1, 16, 48, 1100, 512, 64, 8)])
def test_reference_lcg_case_tiled_bound(O, mlxq_dev, KV, nRep, L, N, D, gs, bits):
    """tests/fused-sdpa.test.ts's five cases (single / multi tile, kv4 and
    kv8, no GQA, the 12B full-attention shape): our prefill vs the
    reference's tiled restatement within its 2/128 bound, on its LCG data."""
    from mlxq import ops

    H = KV * nRep
    bf = O.BF16
    q = O.round_t(O.lcg_floats(H * L * D, 17).reshape(1, H, L, D), bf)
    k = O.round_t(O.lcg_floats(KV * N * D, 18).reshape(1, KV, N, D), bf)
    v = O.round_t(O.lcg_floats(KV * N * D, 19).reshape(1, KV, N, D), bf)
    kq, vq = O.quantize(k, gs, bits, bf), O.quantize(v, gs, bits, bf)
    got = run(O, mlxq_dev, q, kq, vq, bf, 0.125, gs, bits, mask=ops.Mask("causal"))
    tiled = O.sdpa_tiled_t(q, kq, vq, scale=0.125, gs=gs, bits=bits, dtype=bf, causal=True)
    assert np.abs(got - tiled).max() <= 2 / 128
    check(O, got, q, kq, vq, bf, 0.125, gs, bits, "lcg case", causal=True)


@pytest.mark.parametrize("site", [(4, 2, 256, 64, 4), (4, 2, 256, 64, 8), (16, 1, 512, 64, 4)])
def test_reference_decode_sites_vs_unfused(O, mlxq_dev, site):
    """tests/fused-decode-kernel.test.ts:30-67: its randBf16 data, N = 333, the
    12B's three dispatch-site shapes; bounded divergence < 0.02 from the
    unfused path and non-trivial outputs."""
    H, KV, D, gs, bits = site
    N = 333
    bf = O.BF16
    mk = O.rand_bf16_ref
    q, k, v = mk((1, H, 1, D), 11), mk((1, KV, N, D), 22), mk((1, KV, N, D), 33)
    kq, vq = O.quantize(k, gs, bits, bf), O.quantize(v, gs, bits, bf)
    got = run(O, mlxq_dev, q, kq, vq, bf, 1.0, gs, bits)
    un = O.sdpa_unfused_t(q, kq, vq, scale=1.0, gs=gs, bits=bits, dtype=bf)
    assert np.abs(got - un).max() < 0.02
    assert np.abs(un).mean() > 0.001
    check(O, got, q, kq, vq, bf, 1.0, gs, bits, "site")


def test_prefill_full_size_sampled_rows(O, mlxq_dev):
    """The chunked-prefill workload at full size (Lq = 2048 queries at offset
    30720 into a 32768-key 4-bit cache, Hq=32, Hkv=8, D=128, causal): the
    whole launch runs on the GPU; sampled query rows are checked against the
    oracle, where causal row i attends exactly keys [0, 30720 + i] (an
    unmasked oracle call over that prefix)."""
    from mlxq import ops

    B, Hq, Hkv, L, N, D, gs, bits = 1, 32, 8, 2048, 32768, 128, 64, 4
    q, kq, vq = case(O, B, Hq, Hkv, L, N, D, gs, bits, BF16, 21)
    scale = D ** -0.5
    got = run(O, mlxq_dev, q, kq, vq, BF16, scale, gs, bits, mask=ops.Mask("causal"))
    assert got.shape == (B, Hq, L, D) and np.isfinite(got).all()
    for i in (0, 1, 63, 64, 511, 1024, 2046, 2047):
        n = N - L + i + 1
        pre = lambda t: tuple(a[:, :, :n] for a in t)
        ref = O.sdpa(q[:, :, i:i + 1], pre(kq), pre(vq), scale=scale, gs=gs, bits=bits, dtype=BF16)
        assert_close(got[:, :, i:i + 1], ref, what=f"prefill row {i}", dtype=BF16)


@pytest.mark.parametrize("B,Hq,Hkv,L,N,D,gs,bits,dtype,window", [
    (1, 8, 2, 40, 300, 128, 64, 8, BF16, 0),    # 8-bit
    (2, 4, 4, 17, 129, 128, 32, 4, F16, 0),     # fp16, group 32, no GQA, batch 2
    (1, 16, 2, 70, 500, 128, 128, 4, BF16, 0),  # group 128, nRep 8
    (1, 8, 1, 33, 257, 64, 32, 8, F16, 0),      # D = 64
    (1, 4, 2, 65, 400, 64, 64, 8, BF16, 37),    # D = 64, window
    (1, 8, 2, 300, 300, 128, 64, 4, F16, 0),    # prompt: queries = all keys
])
def test_prefill_mfma_variants(O, mlxq_dev, B, Hq, Hkv, L, N, D, gs, bits, dtype, window):
    """Every (D, group_size, bits, dtype) instance family of the MFMA prefill
    kernel against the oracle, bottom-right causal (+ window)."""
    from mlxq import ops

    q, kq, vq = case(O, B, Hq, Hkv, L, N, D, gs, bits, dtype, 70 + L)
    mask = ops.createCausalMask(L, N - L, window or None)
    scale = 1.0 if window else D ** -0.5
    got = run(O, mlxq_dev, q, kq, vq, dtype, scale, gs, bits, mask=mask)
    check(O, got, q, kq, vq, dtype, scale, gs, bits, "prefill variant", causal=True, window=window)


@pytest.mark.parametrize("Hq,Hkv,L,N,D,gs,bits,dtype", [
    (8, 2, 70, 600, 128, 64, 4, BF16),
    (8, 2, 40, 300, 128, 32, 8, F16),   # four groups: two bias MFMAs per block
    (4, 4, 33, 200, 64, 32, 4, BF16),
])
def test_prefill_unscaled_scores(O, mlxq_dev, Hq, Hkv, L, N, D, gs, bits, dtype):
    """Scale 1 on unit-normal q and k (Gemma4 applies no score scale, its q/k
    being RMS-normed: src/model/gemma4-base.ts:1282-1285): |q.k| ~ sqrt(D),
    softmax peaky, so a K dequantized to T before the score product would
    move scores by ~1e-2 and outputs past the bar; the kernel's scores carry
    no rounding of K."""
    from mlxq import ops

    q, kq, vq = case(O, 1, Hq, Hkv, L, N, D, gs, bits, dtype, 90 + L)
    got = run(O, mlxq_dev, q, kq, vq, dtype, 1.0, gs, bits, mask=ops.createCausalMask(L, N - L, None))
    check(O, got, q, kq, vq, dtype, 1.0, gs, bits, "prefill scale 1", causal=True)


@pytest.mark.parametrize("B,Hq,Hkv,L,N,D,gs,bits,dtype,scale,ring", [
    (2, 4, 2, 5, 300, 128, 64, 4, BF16, 1.0, False),   # per-row masks, GQA 2
    (1, 8, 2, 1, 77, 64, 32, 8, F16, 0.125, False),     # decode, one mask for the batch
    (2, 4, 4, 3, 64, 128, 64, 4, BF16, 1.0, True),      # ring rows: keys in temporal order
])
def test_array_mask(O, mlxq_dev, B, Hq, Hkv, L, N, D, gs, bits, dtype, scale, ring):
    """A general "array" mask (neither causal nor a window: the reference's
    where(mask, scores, FINFO_MIN), gemma4-base.ts:1320-1327) against the
    float64 oracle, with a query that attends one key and one that attends
    none (the mean of V over the row's keys)."""
    from mlxq import ops

    q, kq, vq = case(O, B, Hq, Hkv, L, N, D, gs, bits, dtype, 60 + L)
    r = np.random.default_rng(61 + L)
    shape = (B, 1, L, N) if B > 1 else (L, N)
    m = r.random(shape) < 0.4
    flat = m.reshape(-1, L, N)
    flat[0, 0, :] = False
    flat[0, 0, N // 3] = True
    if L > 1:
        flat[-1, L - 1, :] = False
    geo = {}
    if ring:
        geo = dict(valid_len=np.array([N, N - 20], np.int32), ring_off=np.array([17, 50], np.int32))
    got = run(O, mlxq_dev, q, kq, vq, dtype, scale, gs, bits, mask=ops.Mask("array", m),
              valid=geo.get("valid_len"), ring=geo.get("ring_off"))
    ref = O.sdpa_array_mask(q, kq, vq, m, scale=scale, gs=gs, bits=bits, dtype=dtype, **geo)
    assert_close(got, ref, what="array mask", dtype=dtype)


def test_array_mask_shape_errors(O, mlxq_dev):
    """Masks that do not broadcast to [B, 1, L, keys] are rejected on the host."""
    from mlxq import ops

    q, kq, vq = case(O, 2, 4, 2, 3, 40, 64, 64, 4, BF16, 70)
    for bad in (np.ones((2, 40), bool), np.ones((3, 30), bool), np.ones((2, 2, 3, 40), bool)):
        with pytest.raises(ValueError):
            run(O, mlxq_dev, q, kq, vq, BF16, 1.0, 64, 4, mask=ops.Mask("array", bad))

