"""GPU: a quantized checkpoint directory (safetensors + config.json
quantization block) loaded into device arrays and run through the layer
classes: QuantizedEmbedding.encode / asLinear and QuantizedSwitchLinear."""
import json

import numpy as np
import pytest

from conftest import assert_close, write_safetensors

pytestmark = pytest.mark.gpu

BF16 = 12


def test_checkpoint_layers(O, mlxq_dev, tmp_path):
    from mlxq.array import DeviceArray
    from mlxq.weights import (Weights, load_quantized_embedding, load_quantized_switch_linear,
                              read_config_quantization)

    r = np.random.default_rng(5)
    rt = lambda shape, scale=1.0: O.round_t(r.standard_normal(shape).astype(np.float32) * scale, BF16)
    emb_w = rt((512, 256))
    ep, es, eb = O.quantize(emb_w, 64, 8, BF16)           # per-layer override: 8-bit
    exp_w = rt((4, 96, 256), 0.05)
    xp, xs, xb = O.quantize(exp_w, 32, 4, BF16)           # default: 4-bit group 32
    tensors = {
        "model.embed_tokens.weight": ("U32", ep.shape, ep.tobytes()),
        "model.embed_tokens.scales": ("BF16", es.shape, es.tobytes()),
        "model.embed_tokens.biases": ("BF16", eb.shape, eb.tobytes()),
        "model.layers.0.experts.up_proj.weight": ("U32", xp.shape, xp.tobytes()),
        "model.layers.0.experts.up_proj.scales": ("BF16", xs.shape, xs.tobytes()),
        "model.layers.0.experts.up_proj.biases": ("BF16", xb.shape, xb.tobytes()),
    }
    names = list(tensors)
    write_safetensors(str(tmp_path / "model-00001.safetensors"), {k: tensors[k] for k in names[:3]})
    write_safetensors(str(tmp_path / "model-00002.safetensors"), {k: tensors[k] for k in names[3:]})
    with open(tmp_path / "model.safetensors.index.json", "w") as f:
        json.dump({"weight_map": {k: ("model-00001.safetensors" if i < 3 else "model-00002.safetensors")
                                  for i, k in enumerate(names)}}, f)
    with open(tmp_path / "config.json", "w") as f:
        json.dump({"quantization": {"bits": 4, "group_size": 32, "model.embed_tokens": {"bits": 8, "group_size": 64}}},
                  f)

    q = read_config_quantization(str(tmp_path))
    w = Weights(str(tmp_path))
    emb = load_quantized_embedding(w, "model.embed_tokens", q)
    ids = np.array([[3, 511, 0, 42]], np.int32)
    got = emb.encode(DeviceArray.fromNumpy(ids, 7)).toFloat32()
    np.testing.assert_array_equal(got[0], O.dequantize(ep, es, eb, 64, 8, BF16)[ids[0]])

    sw = load_quantized_switch_linear(w, "model.layers.0.experts.up_proj", q)
    x = rt((1, 2, 1, 1, 256))
    idx = np.array([[[2, 0], [3, 1]]], np.uint32)
    y = sw.forward(DeviceArray.fromFloat32(x, x.shape, BF16), DeviceArray.fromNumpy(idx, 3), False).toFloat32()
    assert y.shape == (1, 2, 2, 1, 96)
    deq = lambda e: (O.from_t(xs[e], BF16).astype(np.float64).repeat(32, -1) * O.unpack_codes(xp[e], 4)
                     + O.from_t(xb[e], BF16).astype(np.float64).repeat(32, -1))
    ref = np.stack([x[0, t, 0, 0].astype(np.float64) @ deq(int(idx[0, t, j])).T for t in range(2) for j in range(2)])
    assert_close(y.reshape(4, 96), ref, what="switch linear", dtype=BF16)
    w.dispose()
