"""mlxq -- host mirror of mlx-bun's quantized-inference op surface over
libmlxq, the gfx950 C-ABI library (include/mlxq.h).

    from mlxq import ops, cache
    qt = ops.quantize(w, 64, 4)
    y = ops.quantizedMatmul(x, qt.packed, qt.scales, qt.biases, ops.QuantSpec(4, 64))
    out = ops.quantizedSdpa(q, kq, vq, scale, ops.Mask(""), 64, 4)
"""
from . import cache, ops
from ._lib import MlxqError, ensure_init, synchronize
from .array import DeviceArray, Dtype, bits_to_f32, f32_to_bits

__all__ = ["ops", "cache", "DeviceArray", "Dtype", "MlxqError", "ensure_init", "synchronize",
           "f32_to_bits", "bits_to_f32"]
