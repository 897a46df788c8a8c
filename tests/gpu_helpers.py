"""Shared helpers for the GPU parity tests (calls go through the C ABI)."""
from __future__ import annotations

import ctypes

import numpy as np


def banner(*parts) -> None:
    """Names the case before its device work, so a failing run says what it ran."""
    print("[case]", *parts, flush=True)


def upload_quantized(kt, q):
    """Device QuantizedTensor holding exactly the oracle's packed arrays."""
    return kt.QuantizedTensor(q.qdata, q.scales, q.zeros, (q.rows, q.columns), q.bits, q.group_size)


def gpu_matmul(kt, x: np.ndarray, qt, m: int, c0: np.ndarray | None = None, accumulate: bool = False,
               alpha: float = 1.0) -> np.ndarray:
    a = kt.DeviceBuffer.from_numpy(np.ascontiguousarray(x, dtype=np.float32))
    c = kt.DeviceBuffer(m * qt.columns * 4)
    if c0 is not None:
        c.upload(np.ascontiguousarray(c0, dtype=np.float32))
    else:
        c.fill_zero()
    kt.MatMul.multiply_quantized(a, qt, c, m, accumulate=accumulate, alpha=alpha)
    kt.synchronize()
    return c.download(np.float32).reshape(m, qt.columns)


def gpu_quantize(kt, w: np.ndarray, bits: int, g: int):
    k, n = w.shape
    return kt.QuantizedTensor.quantize(w, k, n, kt.Quantization(bits, g))


def same_bits(a: np.ndarray, b: np.ndarray) -> bool:
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    return a.shape == b.shape and a.tobytes() == b.tobytes()


def raw_ptr(buf, offset: int) -> int:
    return ctypes.c_void_p(buf.ptr + offset).value
