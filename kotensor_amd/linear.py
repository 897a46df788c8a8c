"""``QuantizedLinear``: the drop-in projection holding a device-resident quantized
weight and an fp32 bias (Engine/kotensor/src/main/kotlin/QuantizedLinear.kt:3-46).
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from .device import DeviceBuffer, Stream, default_stream
from .matmul import DeviceTensor
from .quantization import Quantization, QuantizedTensor


class QuantizedLinear:
    """``y = x · deq(W) + bias``; weight ``[inSize x outSize]``."""

    def __init__(self, in_size: int, out_size: int, quantization: Quantization):
        self.in_size = int(in_size)
        self.out_size = int(out_size)
        self.quantization = quantization
        self._weight = QuantizedTensor.empty(in_size, out_size, quantization)
        self.bias = DeviceTensor.zeros((1, out_size))

    @property
    def weight(self) -> QuantizedTensor:
        return self._weight

    @weight.setter
    def weight(self, value: QuantizedTensor) -> None:
        if value.rows != self.in_size or value.columns != self.out_size:
            raise _lib.IllegalArgumentException(
                f"Quantized weight is {value.rows} × {value.columns}, layer is {self.in_size} × {self.out_size}")
        self._weight = value

    def forward(self, x: DeviceTensor, stream: Stream | None = None) -> DeviceTensor:
        """QuantizedLinear.kt:18-20."""
        m = x.shape[0]
        out = DeviceTensor(DeviceBuffer(m * self.out_size * 4), (m, self.out_size))
        return self.forward_into(x, out, stream)

    def forward_into(self, x: DeviceTensor, out: DeviceTensor, stream: Stream | None = None) -> DeviceTensor:
        """QuantizedLinear.kt:22-25: out = x · deq(W), then out += bias, in one launch."""
        if len(x.shape) != 2 or len(out.shape) != 2:
            raise _lib.IllegalArgumentException("not matrices")
        m, k = x.shape
        if k != self._weight.rows:
            raise _lib.IllegalArgumentException(f"{k} != {self._weight.rows}")
        if out.shape != (m, self._weight.columns):
            raise _lib.IllegalArgumentException(f"out shape {list(out.shape)} != [{m}, {self._weight.columns}]")
        _lib.call("kt_qlinear_forward", x.ptr, m, ctypes.byref(self._weight.qweight), self.bias.ptr, out.ptr,
                  (stream or default_stream()).handle)
        return out

    @property
    def size_in_bytes(self) -> int:
        return self._weight.size_in_bytes + self.out_size * 4

    @staticmethod
    def from_linear(weight: np.ndarray, bias: np.ndarray | None, quantization: Quantization) -> "QuantizedLinear":
        """QuantizedLinear.fromLinear, QuantizedLinear.kt:35-40: weight fp32 ``[in x out]``."""
        weight = np.ascontiguousarray(weight, dtype=np.float32)
        in_size, out_size = weight.shape
        layer = QuantizedLinear(in_size, out_size, quantization)
        layer.weight = QuantizedTensor.quantize(weight, in_size, out_size, quantization)
        if bias is not None:
            layer.bias = DeviceTensor.from_numpy(np.asarray(bias, dtype=np.float32).reshape(1, out_size))
        return layer


def forward_into_group(layers, x: DeviceTensor, outs, stream: Stream | None = None):
    """``outs[i] = x · deq(layers[i].weight) + layers[i].bias`` for projections of one input
    (wQ/wK/wV, Attention.kt:220-222; wGate/wUp, SwiGLU.kt:19-25), one launch per four layers."""
    from .matmul import MatMul

    m, k = x.shape
    for layer, out in zip(layers, outs):
        if layer.in_size != k:
            raise _lib.IllegalArgumentException(f"{k} != {layer.in_size}")
        if out.shape != (m, layer.out_size):
            raise _lib.IllegalArgumentException(f"out shape {list(out.shape)} != [{m}, {layer.out_size}]")
    MatMul.multiply_quantized_group(x, [l.weight for l in layers], outs, m, accumulate=False, alpha=1.0,
                                    biases=[l.bias for l in layers], stream=stream)
    return outs


def projection(in_size: int, out_size: int, quantization: Quantization | None):
    """QuantizedLinear.kt:44-46 (only the quantized branch lives on the device)."""
    if quantization is None:
        raise _lib.IllegalArgumentException("only quantized projections run on the HIP path")
    return QuantizedLinear(in_size, out_size, quantization)
