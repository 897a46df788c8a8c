"""saveQuantized files for device-resident weights.

Mirrors ``SafeTensorsFile`` / ``SafeTensors.saveEntries``
(Engine/kotensor/src/main/kotlin/SafeTensors.kt:12-249) and the quantized-weight
parts of ``Transformer.saveQuantized`` / ``loadQuantized`` (Transformer.kt:402-471)
over the C ABI (``kt_st_*``). The file is mapped read-only; a quantized weight's
``.qweight`` / ``.scales`` / ``.zeros`` bytes go straight from the mapping into device
buffers, the layout the kernels consume, with the checks of
``QuantizedTensor.mapFrom`` (QuantizedTensor.kt:109-125). Files written here keep the
reference's header text, padding and entry order, so a file loaded and saved again
is identical byte for byte.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from .device import DeviceBuffer, Stream, default_stream
from .quantization import Quantization, QuantizedTensor, layout

# dtype names of the safetensors header -> numpy dtypes (SafeTensors.kt:22-30)
_DTYPES = {
    "F32": np.float32, "F64": np.float64, "F16": np.float16, "BF16": np.uint16,
    "I8": np.int8, "U8": np.uint8, "BOOL": np.uint8, "I16": np.int16, "U16": np.uint16,
    "I32": np.int32, "U32": np.uint32, "I64": np.int64, "U64": np.uint64,
}


class Entry:
    """``SafeTensorsFile.Entry`` (SafeTensors.kt:14-31)."""

    def __init__(self, name: str, dtype: str, shape, byte_offset: int, byte_length: int):
        self.name = name
        self.dtype = dtype
        self.shape = tuple(int(d) for d in shape)
        self.byte_offset = int(byte_offset)  # from the start of the file
        self.byte_length = int(byte_length)

    @property
    def element_count(self) -> int:
        return int(np.prod(self.shape, dtype=np.int64)) if self.shape else 1

    @property
    def bytes_per_element(self) -> int:
        if self.dtype not in _DTYPES:
            raise _lib.IllegalArgumentException(f"Unsupported safetensors dtype '{self.dtype}' for tensor {self.name}")
        return np.dtype(_DTYPES[self.dtype]).itemsize


class SafeTensorsFile:
    """A read-only mapping of a safetensors file (``SafeTensorsFile``, SafeTensors.kt:12-107)."""

    def __init__(self, path):
        self.path = str(path)
        handle = ctypes.c_void_p()
        _lib.call("kt_st_open", self.path.encode(), ctypes.byref(handle))
        self._h = handle.value
        count = ctypes.c_int32()
        _lib.call("kt_st_count", self._h, ctypes.byref(count))
        buf = ctypes.create_string_buffer(4096)
        self.entries: dict[str, Entry] = {}
        for i in range(count.value):
            _lib.call("kt_st_name", self._h, i, buf, len(buf))
            name = buf.value.decode()
            info = _lib.StEntry()
            _lib.call("kt_st_find", self._h, name.encode(), ctypes.byref(info))
            self.entries[name] = Entry(name, info.dtype.decode(), list(info.shape[:info.rank]), info.offset, info.nbytes)
        self.metadata: dict[str, str] = {}
        lib = _lib.lib()
        i = 0
        while lib.kt_st_metadata_key(self._h, i, buf, len(buf)) == _lib.KT_OK:
            key = buf.value.decode()
            value = ctypes.create_string_buffer(1 << 16)
            _lib.call("kt_st_metadata", self._h, key.encode(), value, len(value))
            self.metadata[key] = value.value.decode()
            i += 1

    # -- lookups (SafeTensors.kt:69-75) -------------------------------------------
    @property
    def names(self) -> list[str]:
        return list(self.entries)

    def __contains__(self, name: str) -> bool:
        return name in self.entries

    def entry(self, name: str) -> Entry:
        if name not in self.entries:
            raise _lib.IllegalArgumentException(f"No tensor named '{name}' in {self.path}")
        return self.entries[name]

    # -- raw and converted reads (SafeTensors.kt:77-137) ---------------------------
    def map(self, name: str) -> np.ndarray:
        """The entry's bytes inside the mapping, without a copy (valid until close)."""
        data = ctypes.c_void_p()
        nbytes = ctypes.c_int64()
        _lib.call("kt_st_data", self._h, name.encode(), ctypes.byref(data), ctypes.byref(nbytes))
        if nbytes.value == 0:
            return np.zeros(0, dtype=np.uint8)
        raw = (ctypes.c_uint8 * nbytes.value).from_address(data.value)
        return np.frombuffer(raw, dtype=np.uint8)

    def read_raw(self, name: str) -> np.ndarray:
        return self.map(name).copy()

    def load(self, name: str) -> np.ndarray:
        """``load(name)``: the entry as fp32 of its shape, converted as ``convert`` does
        (SafeTensors.kt:139-178): BF16 by its upper bits, integers by value."""
        e = self.entry(name)
        count = e.element_count
        if e.byte_length != count * e.bytes_per_element:
            raise _lib.IllegalArgumentException(
                f"Tensor {name} has {e.byte_length} bytes for {count} {e.dtype} elements")
        raw = self.map(name).view(_DTYPES[e.dtype])
        if e.dtype == "BF16":
            out = (raw.astype(np.uint32) << 16).view(np.float32)
        else:
            out = raw.astype(np.float32)
        return out.reshape(e.shape)

    def load_quantized(self, name: str, quantization: Quantization, rows: int, columns: int,
                       stream: Stream | None = None) -> QuantizedTensor:
        """The quantized weight ``name`` (its ``.qweight``, ``.scales`` and ``.zeros``
        entries) in fresh device buffers, checked as ``QuantizedTensor.mapFrom``
        (QuantizedTensor.kt:109-125) checks it."""
        has_zeros = quantization.bits == 4 or f"{name}.zeros" in self.entries
        groups, _, bpr, _ = layout(rows, columns, quantization.bits, quantization.group_size, has_zeros)
        q = DeviceBuffer(rows * bpr)
        s = DeviceBuffer(groups * columns * 4)
        z = DeviceBuffer(groups * columns) if has_zeros else None
        struct = _lib.QWeight(q.ptr, s.ptr, z.ptr if z else None, rows, columns, quantization.bits,
                              quantization.group_size)
        _lib.call("kt_st_load_qweight", self._h, name.encode(), ctypes.byref(struct),
                  (stream or default_stream()).handle)
        return QuantizedTensor(q, s, z, (rows, columns), quantization.bits, quantization.group_size, stream)

    def close(self) -> None:
        if self._h:
            _lib.call("kt_st_close", self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class _Writer:
    def __init__(self):
        handle = ctypes.c_void_p()
        _lib.call("kt_st_writer_create", ctypes.byref(handle))
        self._h = handle.value
        self._keep = []  # host arrays referenced until save

    def metadata(self, key: str, value: str) -> None:
        _lib.call("kt_st_writer_metadata", self._h, key.encode(), str(value).encode())

    def add(self, name: str, dtype: str, shape, data) -> None:
        shape_arr = (ctypes.c_int64 * max(1, len(shape)))(*[int(d) for d in shape])
        if isinstance(data, DeviceBuffer):
            _lib.call("kt_st_writer_add", self._h, name.encode(), dtype.encode(), len(shape), shape_arr, data.ptr,
                      data.nbytes, 1)
        else:
            arr = np.ascontiguousarray(data)
            self._keep.append(arr)
            _lib.call("kt_st_writer_add", self._h, name.encode(), dtype.encode(), len(shape), shape_arr,
                      arr.ctypes.data if arr.nbytes else None, arr.nbytes, 0)
        self._keep.append(shape_arr)

    def add_quantized(self, name: str, weight: QuantizedTensor) -> None:
        _lib.call("kt_st_writer_add_qweight", self._h, name.encode(), ctypes.byref(weight.qweight))

    def save(self, path, stream: Stream | None = None) -> None:
        _lib.call("kt_st_writer_save", self._h, str(path).encode(), (stream or default_stream()).handle)

    def close(self) -> None:
        if self._h:
            _lib.call("kt_st_writer_destroy", self._h)
            self._h = None


def save_entries(path, entries, metadata: dict | None = None, stream: Stream | None = None) -> None:
    """``SafeTensors.saveEntries`` (SafeTensors.kt:204-249). ``entries`` is a sequence of
    ``(name, dtype, shape, data)`` with data a host array or a DeviceBuffer."""
    w = _Writer()
    try:
        for k, v in (metadata or {}).items():
            w.metadata(k, v)
        for name, dtype, shape, data in entries:
            w.add(name, dtype, shape, data)
        w.save(path, stream)
    finally:
        w.close()


def save_quantized(path, parameters: dict, quantized: dict, metadata: dict, stream: Stream | None = None) -> None:
    """The entries ``Transformer.saveQuantized`` writes (Transformer.kt:402-430): the F32
    ``parameters`` (host arrays) in order, then for each quantized weight NAME its
    NAME.qweight, NAME.scales and, with zero points, NAME.zeros, from device memory.
    ``metadata`` holds the kotensor.* keys in the caller's order."""
    w = _Writer()
    try:
        for k, v in metadata.items():
            w.metadata(k, v)
        for name, value in parameters.items():
            arr = np.ascontiguousarray(value, dtype=np.float32)
            w.add(name, "F32", arr.shape, arr)
        for name, weight in quantized.items():
            w.add_quantized(name, weight)
        w.save(path, stream)
    finally:
        w.close()


def load_quantized(path, stream: Stream | None = None):
    """The tensors ``Transformer.loadQuantized`` reads (Transformer.kt:436-471), without
    building a model: returns ``(metadata, parameters, quantized)`` where parameters are
    the F32 entries as host arrays and quantized maps each NAME with a NAME.qweight entry
    to a device ``QuantizedTensor`` of the file's Quantization (kotensor.quantization.*
    metadata)."""
    with SafeTensorsFile(path) as f:
        meta = f.metadata

        def value(key: str) -> str:
            if key not in meta:
                raise _lib.IllegalArgumentException(
                    f"{path} has no {key} metadata; was it written by saveQuantized?")
            return meta[key]

        q = Quantization(int(value("kotensor.quantization.bits")), int(value("kotensor.quantization.groupSize")))
        quantized = {}
        parameters = {}
        suffixes = (".qweight", ".scales", ".zeros")
        for name in f.names:
            if name.endswith(".qweight"):
                base = name[: -len(".qweight")]
                rows = f.entry(name).shape[0]
                columns = f.entry(f"{base}.scales").shape[1]
                quantized[base] = f.load_quantized(base, q, rows, columns, stream)
            elif not name.endswith(suffixes):
                parameters[name] = f.load(name)
        return dict(meta), parameters, quantized
