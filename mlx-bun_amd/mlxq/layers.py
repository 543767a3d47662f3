"""The quantized layer classes of src/model/gemma4-base.ts over libmlxq.

QuantizedEmbedding (:167-201): encode gathers and dequantizes rows of the
packed table in one pass (mlxq_embedding_gather); asLinear is the tied head,
a quantized_matmul against the same table.  QuantizedSwitchLinear
(:1615-1645): the MoE expert projection, gather_qmm over stacked experts.
"""
from __future__ import annotations

from typing import Optional

import numpy as np

from . import _lib, ops
from .array import DeviceArray


class QuantizedEmbedding:
    def __init__(self, w: DeviceArray, scales: DeviceArray, biases: Optional[DeviceArray], spec: ops.QuantSpec):
        self.w, self.scales, self.biases, self.spec = w, scales, biases, spec

    def encode(self, ids: DeviceArray) -> DeviceArray:
        """ids [1, L] (int32 or uint32) -> embeddings [1, L, hidden]; an id
        outside the vocabulary gives a zero row."""
        if self.biases is None:
            raise ValueError("affine embedding requires biases")
        if ids.dtype not in (3, 7):
            raise ValueError("ids must be uint32 or int32")
        for a, n in ((ids, "ids"), (self.w, "weight"), (self.scales, "scales"), (self.biases, "biases")):
            ops._need_contiguous(a, n)
        vocab = self.w.shape[0]
        dim = self.w.shape[-1] * 32 // self.spec.bits
        out = DeviceArray.empty(tuple(ids.shape) + (dim,), self.scales.dtype)
        n = int(np.prod(ids.shape)) if ids.shape else 1
        _lib.call("mlxq_embedding_gather", ids.ptr, n, self.w.ptr, self.scales.ptr, self.biases.ptr,
                  self.scales.dtype, vocab, dim, self.spec.groupSize, self.spec.bits, out.ptr, None)
        return out

    def asLinear(self, h: DeviceArray) -> DeviceArray:
        """Tied output head: h [1, L, hidden] -> logits [1, L, vocab]."""
        return ops.quantizedMatmul(h, self.w, self.scales, self.biases, self.spec, True)


class QuantizedSwitchLinear:
    def __init__(self, w: DeviceArray, scales: DeviceArray, biases: Optional[DeviceArray], spec: ops.QuantSpec):
        self.w, self.scales, self.biases, self.spec = w, scales, biases, spec

    def forward(self, x: DeviceArray, indices: DeviceArray, sortedIndices: bool) -> DeviceArray:
        return ops.gatherQmm(x, self.w, self.scales, self.biases, indices, self.spec, sortedIndices)
