"""Quantized checkpoints on disk -> device arrays.

Mirrors the reference's load path: the safetensors reader
(src/safetensors.ts: [u64 LE header length][JSON header][data], tensors
addressed by byte range, sharded through model.safetensors.index.json), the
Weights map of lazily materialised tensors (src/weights.ts), the
quantization block of config.json (src/config.ts:106-135: a default
{bits, group_size, mode} plus per-module overrides, `false` meaning
unquantized) and the `.load` constructors of the quantized layer classes
(src/model/gemma4-base.ts:175-183, :1623-1639).  Tensor bytes are read
through a read-only memory map and copied to the device on first use; MLX's
packed layout (uint32 words, T scales/biases) is used as stored.
"""
from __future__ import annotations

import json
import os
import struct
from dataclasses import dataclass, field
from typing import Dict, Optional

import numpy as np

from . import ops
from .array import DeviceArray, Dtype

# safetensors dtype -> (bytes per element, numpy storage, mlx dtype code)
_DTYPES = {
    "BOOL": (1, np.uint8, Dtype.bool_), "U8": (1, np.uint8, Dtype.uint8), "I8": (1, np.int8, Dtype.int8),
    "U16": (2, np.uint16, Dtype.uint16), "I16": (2, np.int16, Dtype.int16),
    "U32": (4, np.uint32, Dtype.uint32), "I32": (4, np.int32, Dtype.int32),
    "U64": (8, np.uint64, Dtype.uint64), "I64": (8, np.int64, Dtype.int64),
    "F16": (2, np.uint16, Dtype.float16), "BF16": (2, np.uint16, Dtype.bfloat16),
    "F32": (4, np.float32, Dtype.float32), "F64": (8, np.float64, Dtype.float64),
}


@dataclass
class TensorInfo:
    name: str
    dtype: str
    shape: tuple
    begin: int  # byte range relative to the data section
    end: int


class SafetensorsFile:
    """One safetensors file, memory-mapped read-only (src/safetensors.ts:31-106)."""

    def __init__(self, path: str):
        self.path = path
        size = os.path.getsize(path)
        if size < 8:
            raise ValueError(f"{path}: too small for safetensors")
        with open(path, "rb") as f:
            (header_len,) = struct.unpack("<Q", f.read(8))
            if 8 + header_len > size:
                raise ValueError(f"{path}: header length {header_len} exceeds file size")
            header = json.loads(f.read(header_len).decode("utf-8"))
        self._data_start = 8 + header_len
        self.metadata: Dict[str, str] = {}
        self.tensors: Dict[str, TensorInfo] = {}
        for name, entry in header.items():
            if name == "__metadata__":
                self.metadata = dict(entry)
                continue
            dtype, shape = entry["dtype"], tuple(int(d) for d in entry["shape"])
            begin, end = (int(v) for v in entry["data_offsets"])
            if dtype not in _DTYPES:
                raise ValueError(f"{path}: tensor {name} has unsupported dtype {dtype}")
            expected = int(np.prod(shape)) * _DTYPES[dtype][0] if shape else _DTYPES[dtype][0]
            if begin < 0 or end < begin:
                raise ValueError(f"{path}: tensor {name} has data_offsets [{begin}, {end}] out of order")
            if end - begin != expected:
                raise ValueError(f"{path}: tensor {name} byte range {end - begin} != shape {list(shape)} x {dtype}")
            if self._data_start + end > size:
                raise ValueError(f"{path}: tensor {name} extends past end of file")
            self.tensors[name] = TensorInfo(name, dtype, shape, begin, end)
        self._map = np.memmap(path, dtype=np.uint8, mode="r") if size > self._data_start else None

    def info(self, name: str) -> TensorInfo:
        t = self.tensors.get(name)
        if t is None:
            raise KeyError(f"{self.path}: no tensor named {name}")
        return t

    def view(self, name: str) -> np.ndarray:
        """The tensor's bytes (a view into the mapping)."""
        t = self.info(name)
        if t.end == t.begin:
            return np.zeros(0, np.uint8)
        return self._map[self._data_start + t.begin:self._data_start + t.end]

    def array(self, name: str) -> np.ndarray:
        """The tensor in its storage type (bf16/f16 as raw uint16)."""
        t = self.info(name)
        return self.view(name).view(_DTYPES[t.dtype][1]).reshape(t.shape)


class ShardedSafetensors:
    """A model directory: model.safetensors.index.json + shards, or one
    model.safetensors (src/safetensors.ts:109-161)."""

    def __init__(self, model_dir: str):
        self.files: Dict[str, SafetensorsFile] = {}
        self.tensor_to_file: Dict[str, SafetensorsFile] = {}
        index = os.path.join(model_dir, "model.safetensors.index.json")
        if os.path.exists(index):
            with open(index) as f:
                weight_map = json.load(f)["weight_map"]
            root = os.path.realpath(model_dir)
            for tensor, file in weight_map.items():
                sf = self.files.get(file)
                if sf is None:
                    path = os.path.realpath(os.path.join(model_dir, file))
                    if os.path.commonpath([root, path]) != root:
                        raise ValueError(f"{index}: shard {file!r} of {tensor} lies outside the model directory")
                    sf = self.files[file] = SafetensorsFile(path)
                self.tensor_to_file[tensor] = sf
        else:
            sf = SafetensorsFile(os.path.join(model_dir, "model.safetensors"))
            self.files["model.safetensors"] = sf
            for name in sf.tensors:
                self.tensor_to_file[name] = sf

    @property
    def tensor_names(self):
        return sorted(self.tensor_to_file)

    def _file(self, name: str) -> SafetensorsFile:
        sf = self.tensor_to_file.get(name)
        if sf is None:
            raise KeyError(f"no tensor named {name}")
        return sf

    def info(self, name: str) -> TensorInfo:
        return self._file(name).info(name)

    def array(self, name: str) -> np.ndarray:
        return self._file(name).array(name)


# ------------------------------------------------------------ quantization

@dataclass
class QuantizationConfig:
    default: ops.QuantSpec
    per_layer: Dict[str, ops.QuantSpec] = field(default_factory=dict)


def parse_quantization(raw: Optional[dict]) -> Optional[QuantizationConfig]:
    """config.json's quantization (or quantization_config) block
    (src/config.ts:106-129): bits / group_size / mode defaults, per-module
    objects overriding them, `false` marking a module unquantized."""
    if not raw:
        return None
    default = ops.QuantSpec(raw["bits"], raw["group_size"], raw.get("mode", "affine"))
    per = {}
    for key, value in raw.items():
        if key in ("bits", "group_size", "mode"):
            continue
        if isinstance(value, dict):
            per[key] = ops.QuantSpec(value.get("bits", default.bits), value.get("group_size", default.groupSize),
                                     value.get("mode", default.mode))
        elif value is False:
            per[key] = ops.QuantSpec(0, 0, "none")
    return QuantizationConfig(default, per)


def quant_for(q: Optional[QuantizationConfig], module_path: str) -> Optional[ops.QuantSpec]:
    """The quant spec of a module, or None if it is unquantized (src/config.ts:131-135)."""
    if q is None:
        return None
    spec = q.per_layer.get(module_path, q.default)
    return None if spec.mode == "none" else spec


def read_config_quantization(model_dir: str) -> Optional[QuantizationConfig]:
    with open(os.path.join(model_dir, "config.json")) as f:
        raw = json.load(f)
    return parse_quantization(raw.get("quantization") or raw.get("quantization_config"))


# ---------------------------------------------------------------- weights

class Weights:
    """Tensor name -> device array, copied to the device on first use and
    cached (src/weights.ts:23-91)."""

    def __init__(self, model_dir: str):
        self.shards = ShardedSafetensors(model_dir)
        self._arrays: Dict[str, DeviceArray] = {}

    @property
    def tensor_names(self):
        return self.shards.tensor_names

    def has(self, name: str) -> bool:
        return name in self.shards.tensor_to_file

    def info(self, name: str) -> TensorInfo:
        return self.shards.info(name)

    def tensor(self, name: str) -> DeviceArray:
        a = self._arrays.get(name)
        if a is None:
            info = self.shards.info(name)
            a = DeviceArray.fromNumpy(np.ascontiguousarray(self.shards.array(name)), _DTYPES[info.dtype][2])
            self._arrays[name] = a
        return a

    def dispose(self) -> None:
        for a in self._arrays.values():
            a.dispose()
        self._arrays.clear()


def _quantized_parts(weights: Weights, path: str, quant: Optional[QuantizationConfig], what: str):
    if not weights.has(f"{path}.scales"):
        raise ValueError(f"{path}: expected a quantized {what} (no .scales tensor)")
    spec = quant_for(quant, path)
    if spec is None:
        raise ValueError(f"{path}: no quant spec")
    biases = weights.tensor(f"{path}.biases") if weights.has(f"{path}.biases") else None
    return weights.tensor(f"{path}.weight"), weights.tensor(f"{path}.scales"), biases, spec


def load_quantized_embedding(weights: Weights, path: str, quant: Optional[QuantizationConfig]):
    """QuantizedEmbedding.load (src/model/gemma4-base.ts:175-183)."""
    from .layers import QuantizedEmbedding

    return QuantizedEmbedding(*_quantized_parts(weights, path, quant, "embedding"))


def load_quantized_switch_linear(weights: Weights, path: str, quant: Optional[QuantizationConfig]):
    """QuantizedSwitchLinear.load (src/model/gemma4-base.ts:1623-1639)."""
    from .layers import QuantizedSwitchLinear

    return QuantizedSwitchLinear(*_quantized_parts(weights, path, quant, "switch linear"))


def load_quantized_tensor(weights: Weights, path: str, quant: Optional[QuantizationConfig]):
    """(weight, scales, biases, spec) of a quantized linear module (the
    QuantizedLinear weights, src/model/gemma4-base.ts:120-158)."""
    w, s, b, spec = _quantized_parts(weights, path, quant, "linear")
    return ops.QuantizedTensor(w, s, b), spec
