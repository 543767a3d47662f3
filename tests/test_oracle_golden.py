"""The oracle against the reference's own golden vectors (CPU).

goldens/rotating-kvq.{json,bin} (extracted to tests/golden/ by
tests/golden/make_fixtures.py) holds MLX's quantize outputs driven through a
RotatingQuantizedKVCache (8-bit, group 32, bf16, max_size 64):
scripts/regen-rotating-kvq-goldens.ts:51-72, checked the same way as
tests/rotating-kvq.test.ts:64-105 (offset/idx + active triples bit-exact).
tests/fixtures/batched-rotating-golden.json pins the batched ring window.
"""
import json
import os

import numpy as np
import pytest

from conftest import GOLDEN


@pytest.fixture(scope="module")
def golden():
    return np.load(os.path.join(GOLDEN, "rotating_kvq_mechanics.npz"))


def _drive(O, golden, cache_cls):
    max_size, H, D, gs, bits = (int(v) for v in golden["config"])
    cache = cache_cls(max_size, gs, bits)
    checked = 0
    for i, S in enumerate(golden["step_sizes"]):
        k, v = golden[f"step{i}_k"], golden[f"step{i}_v"]
        assert k.shape == (1, H, S, D)
        kt, vt = cache.update_and_fetch(k, v, O.BF16)
        if i in set(golden["checkpoints"].tolist()):
            off, idx = golden[f"cp{i}_offset_idx"]
            assert (cache.offset, cache.ring_idx) == (off, idx), f"step {i}"
            for name, t in (("k", kt), ("v", vt)):
                np.testing.assert_array_equal(t[0], golden[f"cp{i}_{name}_packed"], err_msg=f"step {i} {name} codes")
                np.testing.assert_array_equal(O.from_t(t[1], O.BF16), golden[f"cp{i}_{name}_scales"])
                np.testing.assert_array_equal(O.from_t(t[2], O.BF16), golden[f"cp{i}_{name}_biases"])
            checked += 1
    return checked


def test_inputs_are_bf16_values(O, golden):
    for i in range(len(golden["step_sizes"])):
        for n in ("k", "v"):
            x = golden[f"step{i}_{n}"]
            np.testing.assert_array_equal(O.round_t(x, O.BF16), x)


def test_quantize_and_ring_bit_exact_vs_golden(O, golden):
    from oracle.kvcache import RotatingQuantizedKVCache

    assert _drive(O, golden, RotatingQuantizedKVCache) == 7


def _numpy_quantize(w, gs, bits, rnd, round_scale_first=False):
    """Independent numpy statement of the affine scheme with a pluggable
    rounding rule (used to show which details the golden fixes)."""
    g = w.reshape(-1, gs).astype(np.float32)
    mn, mx = g.min(1), g.max(1)
    n_bins = np.float32((1 << bits) - 1)
    scale = np.maximum((mx - mn) / n_bins, np.float32(1e-7))
    side = np.abs(mn) > np.abs(mx)
    scale = np.where(side, scale, -scale).astype(np.float32)
    edge = np.where(side, mn, mx).astype(np.float32)
    q0 = rnd((edge / scale).astype(np.float32))
    nz = q0 != 0
    scale = np.where(nz, edge / np.where(nz, q0, 1), scale).astype(np.float32)
    bias = np.where(nz, edge, 0).astype(np.float32)
    if round_scale_first:
        u = scale.view(np.uint32).astype(np.uint64)
        scale = (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16).astype(np.uint32).view(np.float32)
    codes = np.clip(rnd(((g - bias[:, None]) / scale[:, None]).astype(np.float32)), 0, n_bins)
    return codes.astype(np.uint32).reshape(w.shape[:-1] + (w.shape[-1],))


def _half_away(x):
    return np.sign(x) * np.floor(np.abs(x) + np.float32(0.5))


def test_golden_fixes_rounding_rule(O, golden):
    """The golden discriminates the rounding details: round-half-away with
    unrounded fp32 scale/bias matches every code of checkpoint 0; half-even
    or a bf16-rounded scale do not (a plausible restatement error fails)."""
    max_size, H, D, gs, bits = (int(v) for v in golden["config"])
    k = golden["step0_k"]  # 48-token prefill: checkpoint 0 holds exactly these rows
    want = O.unpack_codes(golden["cp0_k_packed"], bits)
    np.testing.assert_array_equal(_numpy_quantize(k, gs, bits, _half_away), want)
    assert (_numpy_quantize(k, gs, bits, np.rint) != want).any()
    assert (_numpy_quantize(k, gs, bits, _half_away, round_scale_first=True) != want).any()


def test_dequantized_golden_reconstructs_inputs(O, golden):
    """Dequantizing the golden codes gives back the step inputs to within half
    a quantization step (plus T rounding) -- closed form s*c+b, and the
    group/element indexing of the oracle's dequantize."""
    max_size, H, D, gs, bits = (int(v) for v in golden["config"])
    k = golden["step0_k"]
    sc = O.to_t(golden["cp0_k_scales"], O.BF16)
    bi = O.to_t(golden["cp0_k_biases"], O.BF16)
    deq = O.dequantize(golden["cp0_k_packed"], sc, bi, gs, bits, O.BF16)
    s = np.abs(golden["cp0_k_scales"]).repeat(gs, axis=-1)
    b = np.abs(golden["cp0_k_biases"]).repeat(gs, axis=-1)
    codes = O.unpack_codes(golden["cp0_k_packed"], bits)
    # codes were rounded against the fp32 scale/bias; storage rounds those to
    # bf16 (unit roundoff 2^-8 each) and the result is rounded to bf16 once more
    bound = 0.5 * s + (codes * s + b + np.abs(deq)) * 2.0 ** -8 + 1e-7
    err = np.abs(deq - k)
    assert np.all(err <= bound)
    assert err.max() > 0.25 * s.max()  # not vacuous: errors span the step


def test_batched_ring_window_matches_reference_masks(O):
    """A ring row's attended slots, given (valid, ring write index), reproduce
    the reference batched rotating cache's per-step decode masks and its
    temporally ordered keys (tests/batched-rotating.test.ts)."""
    g = json.load(open(os.path.join(GOLDEN, "batched_rotating.json")))
    W, B = g["max_size"], g["B"]
    pre = g["prefill_keys"]
    plen = max(len(p) for p in pre)
    # physical buffer after merge: rows left-padded to the longest prefill
    buf = [[0] * plen for _ in range(B)]
    for b in range(B):
        buf[b][plen - len(pre[b]):] = pre[b]
    for s in range(g["steps"]):
        col = (plen + s) % W  # ring write column of this step
        for b in range(B):
            if col >= len(buf[b]):
                buf[b].append(0)
            buf[b][col] = g["decode_keys"][b][s]
        S = len(buf[0])
        ring_off = (col + 1) % S
        for b in range(B):
            valid = min(len(pre[b]) + s + 1, W)
            mask = O.ring_slot_mask(valid, ring_off, S)
            assert mask.astype(int).tolist() == g["per_step"][s]["mask"][b][0][0], (s, b)
            temporal = [buf[b][(ring_off - valid + j) % S] for j in range(valid)]
            assert temporal == g["per_step"][s]["extracted"][b], (s, b)
