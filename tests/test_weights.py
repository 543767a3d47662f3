"""Checkpoint format (host only): the safetensors reader, sharded index,
quantization block and quantized-layer tensors, on synthetic files written
here.  Cases follow tests/safetensors.test.ts (exact bytes, size-mismatch
rejection, the sharded index) and tests/quantize.test.ts (default +
per-layer overrides, false = unquantized)."""
import json
import struct

import numpy as np
import pytest

from conftest import write_safetensors

BF16, F16 = 12, 9


def test_parses_tensors_and_reads_exact_bytes(tmp_path):
    from mlxq.weights import SafetensorsFile

    a = np.array([1.5, -2.25, 3.125, 0], np.float32)
    b = np.array([0x3F80, 0x4000], np.uint16)  # bf16 raw
    p = str(tmp_path / "f.safetensors")
    write_safetensors(p, {"alpha": ("F32", (2, 2), a.tobytes()), "beta": ("BF16", (2,), b.tobytes())},
                      metadata={"format": "pt"})
    sf = SafetensorsFile(p)
    assert sf.metadata["format"] == "pt"
    assert sorted(sf.tensors) == ["alpha", "beta"]
    assert sf.tensors["alpha"].dtype == "F32" and sf.tensors["alpha"].shape == (2, 2)
    np.testing.assert_array_equal(sf.array("alpha").ravel(), a)
    assert len(sf.view("beta")) == 4
    np.testing.assert_array_equal(sf.array("beta"), b)


def test_rejects_size_mismatch_and_overrun(tmp_path):
    from mlxq.weights import SafetensorsFile

    p = str(tmp_path / "bad.safetensors")
    write_safetensors(p, {"t": ("F32", (3,), np.zeros(2, np.float32).tobytes())})
    with pytest.raises(ValueError, match="byte range"):
        SafetensorsFile(p)
    hb = json.dumps({"t": {"dtype": "F32", "shape": [4], "data_offsets": [0, 16]}}).encode()
    with open(p, "wb") as f:
        f.write(struct.pack("<Q", len(hb)) + hb + b"\0" * 8)  # 8 of the 16 bytes
    with pytest.raises(ValueError, match="past end"):
        SafetensorsFile(p)
    with open(p, "wb") as f:
        f.write(struct.pack("<Q", 1 << 40))
    with pytest.raises(ValueError, match="header length"):
        SafetensorsFile(p)


def test_rejects_negative_or_reversed_offsets(tmp_path):
    """data_offsets must satisfy 0 <= begin <= end (a negative begin would
    read header bytes as tensor data)."""
    from mlxq.weights import SafetensorsFile

    p = str(tmp_path / "neg.safetensors")
    for offs in ([-8, 8], [16, 0]):
        hb = json.dumps({"t": {"dtype": "F32", "shape": [4], "data_offsets": offs}}).encode()
        with open(p, "wb") as f:
            f.write(struct.pack("<Q", len(hb)) + hb + b"\0" * 16)
        with pytest.raises(ValueError, match="out of order"):
            SafetensorsFile(p)


def test_sharded_index_rejects_paths_outside_the_model_dir(tmp_path):
    from mlxq.weights import ShardedSafetensors

    model = tmp_path / "model"
    model.mkdir()
    write_safetensors(str(tmp_path / "outside.safetensors"), {"t": ("F32", (1,), np.zeros(1, np.float32).tobytes())})
    with open(model / "model.safetensors.index.json", "w") as f:
        json.dump({"weight_map": {"t": "../outside.safetensors"}}, f)
    with pytest.raises(ValueError, match="outside the model directory"):
        ShardedSafetensors(str(model))


def test_sharded_index(tmp_path):
    from mlxq.weights import ShardedSafetensors

    vals = {f"t{i}": np.arange(4 * i + 1, 4 * i + 5, dtype=np.float32) for i in range(3)}
    write_safetensors(str(tmp_path / "a.safetensors"), {k: ("F32", (4,), vals[k].tobytes()) for k in ("t0", "t1")})
    write_safetensors(str(tmp_path / "b.safetensors"), {"t2": ("F32", (4,), vals["t2"].tobytes())})
    with open(tmp_path / "model.safetensors.index.json", "w") as f:
        json.dump({"weight_map": {"t0": "a.safetensors", "t1": "a.safetensors", "t2": "b.safetensors"}}, f)
    sh = ShardedSafetensors(str(tmp_path))
    assert sh.tensor_names == ["t0", "t1", "t2"]
    np.testing.assert_array_equal(sh.array("t2"), [9, 10, 11, 12])
    assert len(sh.files) == 2


def test_quantization_block():
    from mlxq.weights import parse_quantization, quant_for

    q = parse_quantization({"bits": 4, "group_size": 64,
                            "model.embed_tokens": {"bits": 8, "group_size": 64},
                            "model.layers.0.self_attn.q_proj": {"bits": 4, "group_size": 32},
                            "model.norm": False})
    assert (q.default.bits, q.default.groupSize, q.default.mode) == (4, 64, "affine")
    e = quant_for(q, "model.embed_tokens")
    assert (e.bits, e.groupSize) == (8, 64)
    assert quant_for(q, "model.layers.0.self_attn.q_proj").groupSize == 32
    assert quant_for(q, "model.norm") is None
    d = quant_for(q, "model.layers.3.mlp.down_proj")
    assert (d.bits, d.groupSize) == (4, 64)
    assert parse_quantization(None) is None and quant_for(None, "x") is None


def test_quantized_layer_tensors_round_trip(tmp_path, O):
    """A 4-bit embedding written as <path>.weight / .scales / .biases reads back
    as MLX's packed layout, byte for byte."""
    from mlxq.weights import ShardedSafetensors, read_config_quantization, quant_for

    w = O.round_t(np.random.default_rng(0).standard_normal((64, 128)).astype(np.float32), BF16)
    p, s, b = O.quantize(w, 64, 4, BF16)
    write_safetensors(str(tmp_path / "model.safetensors"), {
        "model.embed_tokens.weight": ("U32", p.shape, p.tobytes()),
        "model.embed_tokens.scales": ("BF16", s.shape, s.tobytes()),
        "model.embed_tokens.biases": ("BF16", b.shape, b.tobytes()),
    })
    with open(tmp_path / "config.json", "w") as f:
        json.dump({"model_type": "gemma4", "quantization_config": {"bits": 4, "group_size": 64}}, f)
    sh = ShardedSafetensors(str(tmp_path))
    np.testing.assert_array_equal(sh.array("model.embed_tokens.weight"), p)
    np.testing.assert_array_equal(sh.array("model.embed_tokens.scales"), s)
    np.testing.assert_array_equal(sh.array("model.embed_tokens.biases"), b)
    spec = quant_for(read_config_quantization(str(tmp_path)), "model.embed_tokens")
    assert (spec.bits, spec.groupSize) == (4, 64)
