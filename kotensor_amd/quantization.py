"""Quantization scheme and device-resident quantized tensor.

Mirrors ``Quantization`` and ``QuantizedTensor``
(Engine/kotensor/src/main/kotlin/QuantizedTensor.kt:10-326): same fields, same
derived layout numbers, same validation messages, and the reference's packed
layout kept byte for byte (qdata ``[rows x bytesPerRow]``, scales
``[groups x columns]`` fp32, zeros ``[groups x columns]``). The arrays live in
device memory; reading ``qdata`` / ``scales`` / ``zeros`` copies them back, as the
reference's getters move mapped data to the heap.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from .device import DeviceBuffer, Stream, default_stream


class Quantization:
    """``Quantization(bits, groupSize = 64)``, QuantizedTensor.kt:10-25."""

    def __init__(self, bits: int, group_size: int = 64):
        if bits not in (4, 8):
            raise _lib.IllegalArgumentException(f"bits must be 4 or 8, got {bits}")
        if group_size <= 0:
            raise _lib.IllegalArgumentException("groupSize must be positive")
        self.bits = int(bits)
        self.group_size = int(group_size)

    def __str__(self) -> str:
        return f"int{self.bits}/g{self.group_size}"

    __repr__ = __str__


Quantization.INT8 = Quantization(8)
Quantization.INT4 = Quantization(4)


def layout(rows: int, columns: int, bits: int, group_size: int, has_zeros: bool) -> tuple[int, int, int, int]:
    """(groups, storedColumns, bytesPerRow, sizeInBytes), QuantizedTensor.kt:47-49,97-98."""
    out = (ctypes.c_int64 * 4)()
    _lib.call("kt_qweight_layout", rows, columns, bits, group_size, int(bool(has_zeros)), out)
    return int(out[0]), int(out[1]), int(out[2]), int(out[3])


class QuantizedTensor:
    """A quantized ``[rows x columns]`` weight (rows = K inputs, columns = N outputs)."""

    def __init__(self, qdata, scales, zeros, shape, bits: int, group_size: int,
                 stream: Stream | None = None):
        shape = tuple(int(d) for d in shape)
        if len(shape) != 2 or shape[0] <= 0 or shape[1] <= 0:
            raise _lib.IllegalArgumentException(f"QuantizedTensor needs a 2-D shape, got {list(shape)}")
        if bits not in (4, 8):
            raise _lib.IllegalArgumentException("bits must be 4 or 8")
        self.shape = shape
        self.bits = int(bits)
        self.group_size = int(group_size)
        self.has_zero_points = zeros is not None
        self.groups, self.stored_columns, self.bytes_per_row, self.size_in_bytes = layout(
            shape[0], shape[1], bits, group_size, self.has_zero_points)
        self._q = self._adopt(qdata, self.rows * self.bytes_per_row, np.uint8, "qdata", "bytes", stream)
        self._s = self._adopt(scales, self.groups * self.columns, np.float32, "scales", "entries", stream)
        self._z = None if zeros is None else self._adopt(zeros, self.groups * self.columns, np.uint8, "zeros",
                                                         "entries", stream)
        if self.bits == 4 and not self.has_zero_points:
            raise _lib.IllegalArgumentException("4-bit tensors need zero points")
        self._p = None
        self._struct = _lib.QWeight(self._q.ptr, self._s.ptr, self._z.ptr if self._z else None,
                                    self.rows, self.columns, self.bits, self.group_size, None)
        _lib.call("kt_qweight_check", ctypes.byref(self._struct))

    @staticmethod
    def _adopt(value, count, dtype, name, unit, stream):
        itemsize = np.dtype(dtype).itemsize
        if isinstance(value, DeviceBuffer):
            if value.nbytes != count * itemsize:
                raise _lib.IllegalArgumentException(
                    f"{name} has {value.nbytes // itemsize} {unit}, expected {count}")
            return value
        arr = np.ascontiguousarray(value)
        if arr.size != count:
            raise _lib.IllegalArgumentException(f"{name} has {arr.size} {unit}, expected {count}")
        return DeviceBuffer.from_numpy(arr.view(dtype) if arr.dtype.itemsize == itemsize else arr.astype(dtype),
                                       stream)

    # -- shape (QuantizedTensor.kt:45-49) ---------------------------------------
    @property
    def rows(self) -> int:
        return self.shape[0]

    @property
    def columns(self) -> int:
        return self.shape[1]

    # -- raw device views used by the kernels -------------------------------------
    @property
    def qweight(self) -> "_lib.QWeight":
        """The ``kt_qweight`` struct passed to the C ABI."""
        return self._struct

    @property
    def qdata_buffer(self) -> DeviceBuffer:
        return self._q

    @property
    def scales_buffer(self) -> DeviceBuffer:
        return self._s

    @property
    def zeros_buffer(self) -> DeviceBuffer | None:
        return self._z

    @property
    def packed_buffer(self) -> DeviceBuffer | None:
        """The column-run copy of qdata written by :meth:`pack`, or None."""
        return self._p

    def pack(self, stream: Stream | None = None) -> "QuantizedTensor":
        """Writes the device-native column-run copy of qdata, scales and zeros
        (``kt_qweight_pack``) and points the weight at it, so one-row products (and, for
        group sizes that are multiples of 32, the prefill GEMM) read it instead of qdata.
        qdata, scales and zeros stay the format of record (files, accessors, the other
        kernels). Costs ``kt_qweight_packed_bytes`` more device memory (about the size of
        qdata plus the scales and zeros); call it again after they change. Returns self."""
        n = ctypes.c_int64()
        _lib.call("kt_qweight_packed_bytes", self.rows, self.columns, self.bits, self.group_size, ctypes.byref(n))
        if self._p is None or self._p.nbytes != n.value:
            self._p = DeviceBuffer(n.value)
        self._struct.packed = None
        _lib.call("kt_qweight_pack", ctypes.byref(self._struct), self._p.ptr, (stream or default_stream()).handle)
        self._struct.packed = self._p.ptr
        return self

    def unpack(self) -> None:
        """Drops the column-run copy (every product reads qdata again)."""
        self._struct.packed = None
        if self._p is not None:
            self._p.free()
            self._p = None

    # -- host copies (QuantizedTensor.kt:72-92) -----------------------------------
    @property
    def qdata(self) -> np.ndarray:
        """Packed bytes as signed int8 (a Kotlin ByteArray), ``rows * bytesPerRow``."""
        return self._q.download(np.int8)

    @property
    def scales(self) -> np.ndarray:
        return self._s.download(np.float32)

    @property
    def zeros(self) -> np.ndarray | None:
        return None if self._z is None else self._z.download(np.int8)

    # -- accessors (QuantizedTensor.kt:172-249) ----------------------------------
    def raw_value(self, row: int, column: int) -> int:
        """Stored integer: signed byte (8-bit) or nibble 0..15 (4-bit), QuantizedTensor.kt:172-180."""
        if self.bits == 8:
            return int(self._q.download(np.int8, 1, offset=row * self.bytes_per_row + column)[0])
        half = self.bytes_per_row
        byte = int(self._q.download(np.uint8, 1, offset=row * self.bytes_per_row + column % half)[0])
        return byte & 0xF if column < half else (byte >> 4) & 0xF

    def value(self, row: int, column: int) -> float:
        """``scale * (raw - zero)``, QuantizedTensor.kt:182-186 (computed on the device)."""
        return float(self.dequantize_column(column)[row])

    def dequantize_rows(self, rows, stream: Stream | None = None) -> np.ndarray:
        """dequantizeRow for each row index, ``[len(rows) x columns]`` (QuantizedTensor.kt:188-213)."""
        idx = np.ascontiguousarray(rows, dtype=np.int32)
        if idx.size and (idx.min() < 0 or idx.max() >= self.rows):
            raise _lib.IllegalArgumentException(f"row out of range for {self.rows} rows")
        dev_idx = DeviceBuffer.from_numpy(idx, stream)
        out = DeviceBuffer(idx.size * self.columns * 4)
        _lib.call("kt_dequantize_rows", ctypes.byref(self._struct), dev_idx.ptr, int(idx.size), out.ptr,
                  (stream or default_stream()).handle)
        return out.download(np.float32, stream=stream).reshape(idx.size, self.columns)

    def dequantize_row(self, row: int) -> np.ndarray:
        return self.dequantize_rows([row])[0]

    def dequantize_column(self, column: int, stream: Stream | None = None) -> np.ndarray:
        """dequantizeColumn, QuantizedTensor.kt:235-241."""
        if not 0 <= column < self.columns:
            raise _lib.IllegalArgumentException(f"column {column} out of range for {self.columns} columns")
        idx = DeviceBuffer.from_numpy(np.array([column], dtype=np.int32), stream)
        out = DeviceBuffer(self.rows * 4)
        _lib.call("kt_dequantize_columns", ctypes.byref(self._struct), idx.ptr, 1, out.ptr,
                  (stream or default_stream()).handle)
        return out.download(np.float32, stream=stream)

    def dequantize(self) -> np.ndarray:
        """The full fp32 ``[rows x columns]`` matrix, QuantizedTensor.kt:243-249."""
        return self.dequantize_rows(np.arange(self.rows, dtype=np.int32))

    # -- quantize (QuantizedTensor.kt:256-324) -----------------------------------
    @staticmethod
    def empty(rows: int, columns: int, quantization: Quantization) -> "QuantizedTensor":
        """All-zero tensor of the scheme's layout (QuantizedTensor.kt:252-254)."""
        groups, _, bpr, _ = layout(rows, columns, quantization.bits, quantization.group_size,
                                   quantization.bits == 4)
        q = DeviceBuffer(rows * bpr)
        s = DeviceBuffer(groups * columns * 4)
        z = DeviceBuffer(groups * columns) if quantization.bits == 4 else None
        for b in (q, s, z):
            if b is not None:
                b.fill_zero()
        return QuantizedTensor(q, s, z, (rows, columns), quantization.bits, quantization.group_size)

    @staticmethod
    def quantize(data, rows: int, columns: int, quantization: Quantization,
                 stream: Stream | None = None) -> "QuantizedTensor":
        """Quantizes fp32 ``data`` (host array or DeviceBuffer, row-major ``[rows x columns]``)
        on the device. Raises IllegalArgumentException where the reference's
        ``roundToInt`` would reject a NaN."""
        if isinstance(data, DeviceBuffer):
            if data.nbytes != rows * columns * 4:
                raise _lib.IllegalArgumentException(
                    f"data has {data.nbytes // 4} elements, expected {rows} × {columns}")
            src = data
        else:
            arr = np.ascontiguousarray(data, dtype=np.float32)
            if arr.size != rows * columns:
                raise _lib.IllegalArgumentException(f"data has {arr.size} elements, expected {rows} × {columns}")
            src = DeviceBuffer.from_numpy(arr, stream)
        groups, _, bpr, _ = layout(rows, columns, quantization.bits, quantization.group_size,
                                   quantization.bits == 4)
        q = DeviceBuffer(rows * bpr)
        s = DeviceBuffer(groups * columns * 4)
        z = DeviceBuffer(groups * columns) if quantization.bits == 4 else None
        _lib.call("kt_quantize", src.ptr, rows, columns, quantization.bits, quantization.group_size, q.ptr, s.ptr,
                  z.ptr if z else None, (stream or default_stream()).handle)
        return QuantizedTensor(q, s, z, (rows, columns), quantization.bits, quantization.group_size)

    def free(self) -> None:
        self.unpack()
        for b in (self._q, self._s, self._z):
            if b is not None:
                b.free()
