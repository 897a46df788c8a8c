"""``fusedCrossEntropyLoss`` with a quantized head
(Engine/kotensor/src/main/kotlin/Loss.kt:114-219) on the device, through
``kt_fused_cross_entropy``.

The reference returns a 1 x 1 loss tensor whose backward closure adds
``upstream * d loss / d hidden`` to ``hidden.grad`` and ``upstream * d loss / d bias`` to
the head's bias gradient. This mirror has no autograd: it returns the loss and, when
asked, writes those gradients for an upstream gradient of 1 (added to what the buffers
hold with ``accumulate``).
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from .device import DeviceBuffer, Stream, default_stream
from .linear import QuantizedLinear
from .matmul import DeviceTensor

IGNORE_INDEX = -100  # Loss.kt:6


class FusedLoss:
    """The result of ``fused_cross_entropy_loss``: the loss on the device, the gradients if
    requested (DeviceTensor or None)."""

    def __init__(self, loss: DeviceBuffer, hidden_grad: DeviceTensor | None, bias_grad: DeviceTensor | None):
        self.loss_buffer = loss
        self.hidden_grad = hidden_grad
        self.bias_grad = bias_grad

    def item(self, stream: Stream | None = None) -> float:
        return float(self.loss_buffer.download(np.float32, stream=stream)[0])


def fused_cross_entropy_loss(hidden: DeviceTensor, head: QuantizedLinear, targets, ignore_index: int = IGNORE_INDEX,
                             grads: bool = True, hidden_grad: DeviceTensor | None = None,
                             bias_grad: DeviceTensor | None = None, accumulate: bool = False,
                             stream: Stream | None = None) -> FusedLoss:
    """Loss.kt:114-219 for a ``QuantizedLinear`` head: hidden [rows x inSize] on the device,
    targets a host sequence of ints (ignore_index skips a row). With ``grads`` the
    gradients go to ``hidden_grad`` / ``bias_grad`` (new zeroed tensors when not given)."""
    t = np.ascontiguousarray(np.asarray(targets, dtype=np.int32).reshape(-1))
    rows = int(t.size)
    if rows == 0:
        raise _lib.IllegalArgumentException("targets cannot be empty")
    if len(hidden.shape) != 2 or hidden.shape != (rows, head.in_size):
        raise _lib.IllegalArgumentException(
            f"hidden has {int(np.prod(hidden.shape))} elements, expected {rows} × {head.in_size}")
    if grads:
        if hidden_grad is None:
            hidden_grad = DeviceTensor.zeros((rows, head.in_size))
        if bias_grad is None:
            bias_grad = DeviceTensor.zeros((1, head.out_size))
        if hidden_grad.shape != (rows, head.in_size) or int(np.prod(bias_grad.shape)) != head.out_size:
            raise _lib.IllegalArgumentException("gradient buffers do not match hidden and the head")
    else:
        hidden_grad = bias_grad = None
    loss = DeviceBuffer(4)
    _lib.call("kt_fused_cross_entropy", hidden.ptr, rows, ctypes.byref(head.weight.qweight), head.bias.ptr,
              t.ctypes.data_as(ctypes.c_void_p), int(ignore_index), loss.ptr,
              hidden_grad.ptr if hidden_grad is not None else None,
              bias_grad.ptr if bias_grad is not None else None, int(bool(accumulate)),
              (stream or default_stream()).handle)
    return FusedLoss(loss, hidden_grad, bias_grad)
