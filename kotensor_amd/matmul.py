"""Dequantizing matmul entry points, mirroring ``MatMul``
(Engine/kotensor/src/main/kotlin/MatMul.kt:460-486 and :954-981), and the
device tensor that ``Tensor.matmulDequant(Into)`` (Tensor.kt:162-188) acts on.

Operands are device buffers; the work is enqueued on a stream and runs in HIP.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from .device import DeviceBuffer, Stream, default_stream
from .quantization import QuantizedTensor


class DeviceTensor:
    """A row-major fp32 matrix in device memory (the data a ``Tensor`` holds)."""

    def __init__(self, buffer: DeviceBuffer, shape):
        shape = tuple(int(d) for d in shape)
        n = int(np.prod(shape)) if shape else 1
        if buffer.nbytes != n * 4:
            raise _lib.IllegalArgumentException(f"buffer of {buffer.nbytes} bytes does not hold {list(shape)} floats")
        self.buffer = buffer
        self.shape = shape

    @classmethod
    def from_numpy(cls, array, stream: Stream | None = None) -> "DeviceTensor":
        arr = np.ascontiguousarray(array, dtype=np.float32)
        if arr.ndim == 1:
            arr = arr.reshape(1, -1)
        return cls(DeviceBuffer.from_numpy(arr, stream), arr.shape)

    @classmethod
    def zeros(cls, shape) -> "DeviceTensor":
        buf = DeviceBuffer(int(np.prod(shape)) * 4)
        buf.fill_zero()
        return cls(buf, shape)

    def numpy(self, stream: Stream | None = None) -> np.ndarray:
        return self.buffer.download(np.float32, stream=stream).reshape(self.shape)

    @property
    def ptr(self) -> int:
        return self.buffer.ptr

    def matmul_dequant(self, weight: QuantizedTensor, stream: Stream | None = None) -> "DeviceTensor":
        """``this · deq(W)`` into a new tensor, Tensor.kt:162-178 (forward only)."""
        if len(self.shape) != 2:
            raise _lib.IllegalArgumentException("not a matrix")
        m, k = self.shape
        if k != weight.rows:
            raise _lib.IllegalArgumentException(f"{k} != {weight.rows}")
        out = DeviceTensor(DeviceBuffer(m * weight.columns * 4), (m, weight.columns))
        MatMul.multiply_quantized(self.buffer, weight, out.buffer, m, accumulate=False, stream=stream)
        return out

    def matmul_dequant_into(self, weight: QuantizedTensor, out: "DeviceTensor", accumulate: bool = False,
                            scale: float = 1.0, stream: Stream | None = None) -> "DeviceTensor":
        """Tensor.kt:180-188."""
        if len(self.shape) != 2 or len(out.shape) != 2:
            raise _lib.IllegalArgumentException("not matrices")
        m, k = self.shape
        if k != weight.rows:
            raise _lib.IllegalArgumentException(f"{k} != {weight.rows}")
        if out.shape != (m, weight.columns):
            raise _lib.IllegalArgumentException(f"out shape {list(out.shape)} != [{m}, {weight.columns}]")
        MatMul.multiply_quantized(self.buffer, weight, out.buffer, m, accumulate, scale, stream)
        return out


def _ptr(x):
    return x.ptr if isinstance(x, (DeviceBuffer, DeviceTensor)) else x


def _nbytes(x):
    if isinstance(x, DeviceTensor):
        return x.buffer.nbytes
    if isinstance(x, DeviceBuffer):
        return x.nbytes
    return None


class MatMul:
    """The quantized half of ``object MatMul``."""

    @staticmethod
    def multiply_quantized(a, weight: QuantizedTensor, c, m: int, accumulate: bool = True, alpha: float = 1.0,
                           stream: Stream | None = None) -> None:
        """``c[m x N] = (accumulate ? c : 0) + alpha * a[m x K] · deq(W)``, MatMul.kt:460-486."""
        k, n = weight.rows, weight.columns
        if m < 0:
            raise _lib.IllegalArgumentException(f"Negative row count {m}")
        na, nc = _nbytes(a), _nbytes(c)
        if na is not None and na < m * k * 4:
            raise _lib.IllegalArgumentException(f"a has {na // 4} elements, needs {m} × {k}")
        if nc is not None and nc < m * n * 4:
            raise _lib.IllegalArgumentException(f"c has {nc // 4} elements, needs {m} × {n}")
        if m == 0:
            return
        _lib.call("kt_qmatmul", _ptr(a), int(m), ctypes.byref(weight.qweight), _ptr(c), int(bool(accumulate)),
                  ctypes.c_float(alpha), (stream or default_stream()).handle)

    @staticmethod
    def multiply_quantized_group(a, weights, outputs, m: int, accumulate: bool = False, alpha: float = 1.0,
                                 biases=None, stream: Stream | None = None) -> None:
        """Several projections of one input in one call (kt_qmatmul_group): for each i,
        ``outputs[i] = (accumulate ? outputs[i] : 0) + alpha * a · deq(weights[i]) (+ biases[i])``.
        The weights must share rows, bits and group size (q/k/v, gate/up)."""
        count = len(weights)
        if count != len(outputs) or (biases is not None and len(biases) != count):
            raise _lib.IllegalArgumentException("weights, outputs and biases differ in length")
        if count == 0:
            return
        k = weights[0].rows
        na = _nbytes(a)
        if na is not None and na < m * k * 4:
            raise _lib.IllegalArgumentException(f"a has {na // 4} elements, needs {m} × {k}")
        for w, c in zip(weights, outputs):
            nc = _nbytes(c)
            if nc is not None and nc < m * w.columns * 4:
                raise _lib.IllegalArgumentException(f"output has {nc // 4} elements, needs {m} × {w.columns}")
        structs = (_lib.QWeight * count)(*[w.qweight for w in weights])
        outs = (ctypes.c_void_p * count)(*[_ptr(c) for c in outputs])
        bias_arr = None if biases is None else (ctypes.c_void_p * count)(
            *[None if b is None else _ptr(b) for b in biases])
        _lib.call("kt_qmatmul_group", _ptr(a), int(m), structs, count, outs, bias_arr, int(bool(accumulate)),
                  ctypes.c_float(alpha), (stream or default_stream()).handle)

    @staticmethod
    def multiply_by_quantized_transposed(dy, weight: QuantizedTensor, dx, m: int, accumulate: bool = True,
                                         stream: Stream | None = None) -> None:
        """``dx[m x K] = (accumulate ? dx : 0) + dy[m x N] · deq(W)^T``, MatMul.kt:954-981."""
        k, n = weight.rows, weight.columns
        ndy, ndx = _nbytes(dy), _nbytes(dx)
        if ndy is not None and ndy < m * n * 4:
            raise _lib.IllegalArgumentException(f"dy has {ndy // 4} elements, needs {m} × {n}")
        if ndx is not None and ndx < m * k * 4:
            raise _lib.IllegalArgumentException(f"dx has {ndx // 4} elements, needs {m} × {k}")
        if m == 0:
            return
        _lib.call("kt_qmatmul_transposed", _ptr(dy), int(m), ctypes.byref(weight.qweight), _ptr(dx),
                  int(bool(accumulate)), (stream or default_stream()).handle)

    @staticmethod
    def set_kernel_config(gemv_kind: int = 0, gemv_vec: int = 0, gemv_splits: int = 0, gemv_waves: int = 0,
                          gemv_reduce: int = 0) -> None:
        """Work-split knobs of the small-M kernels (the counterpart of MatMul.kt:30-82's knobs)."""
        _lib.call("kt_set_kernel_config", int(gemv_kind), int(gemv_vec), int(gemv_splits), int(gemv_waves),
                  int(gemv_reduce))
