"""The oracle for the saveQuantized file format: a plain-Python restatement of the
reference's safetensors writer and reader.

TEST INFRASTRUCTURE ONLY (the checker of kt_st_*); the product never imports it.

  write_entries  -- SafeTensors.saveEntries + jsonString
                    (Engine/kotensor/src/main/kotlin/SafeTensors.kt:204-265): metadata
                    first as "__metadata__", then one header entry per tensor with
                    data_offsets accumulated in order, the header padded with spaces to a
                    multiple of 8, the size as a little-endian int64, then the data.
  read_header    -- SafeTensorsFile's header parse (SafeTensors.kt:37-67).
  quantized_entries -- the entries Transformer.saveQuantized adds per quantized weight
                    (Transformer.kt:425-428).

Pinning: files from write_entries are read back by the `safetensors` package (an
independent implementation of the format) in the tests, and read_header agrees with
it on every tensor and metadata key.
"""
from __future__ import annotations

import json
import struct

import numpy as np


def json_string(text: str) -> str:
    """jsonString (SafeTensors.kt:251-265)."""
    out = ['"']
    for ch in text:
        if ch == '"':
            out.append('\\"')
        elif ch == "\\":
            out.append("\\\\")
        elif ch == "\n":
            out.append("\\n")
        elif ch == "\r":
            out.append("\\r")
        elif ch == "\t":
            out.append("\\t")
        elif ord(ch) < 0x20:
            out.append("\\u%04x" % ord(ch))
        else:
            out.append(ch)
    out.append('"')
    return "".join(out)


def write_entries(entries, metadata: dict | None = None) -> bytes:
    """The bytes SafeTensors.saveEntries writes. entries: (name, dtype, shape, raw bytes)."""
    parts = []
    if metadata:
        pairs = ",".join(f"{json_string(k)}:{json_string(v)}" for k, v in metadata.items())
        parts.append(f'"__metadata__":{{{pairs}}}')
    offset = 0
    for name, dtype, shape, raw in entries:
        start, end = offset, offset + len(raw)
        dims = ",".join(str(int(d)) for d in shape)
        parts.append(f'{json_string(name)}:{{"dtype":"{dtype}","shape":[{dims}],"data_offsets":[{start},{end}]}}')
        offset = end
    header = ("{" + ",".join(parts) + "}").encode("utf-8")
    padding = (8 - len(header) % 8) % 8
    return struct.pack("<q", len(header) + padding) + header + b" " * padding + b"".join(raw for *_, raw in entries)


def read_header(data: bytes):
    """(entries {name: (dtype, shape, start, end)}, metadata) of a file's bytes."""
    (size,) = struct.unpack_from("<q", data, 0)
    if not 1 <= size <= (100 << 20):
        raise ValueError(f"Invalid safetensors header size {size}")
    header = json.loads(data[8:8 + size].decode("utf-8"))
    entries, metadata = {}, {}
    for name, body in header.items():
        if not isinstance(body, dict):
            continue
        if name == "__metadata__":
            metadata = {k: str(v) for k, v in body.items()}
            continue
        start, end = body["data_offsets"]
        entries[name] = (body["dtype"], tuple(body.get("shape", [])), 8 + size + start, 8 + size + end)
    return entries, metadata


def quantized_entries(name: str, bits: int, rows: int, bytes_per_row: int, groups: int, columns: int,
                      qdata: np.ndarray, scales: np.ndarray, zeros: np.ndarray | None):
    """Transformer.saveQuantized's entries for one weight (Transformer.kt:425-428)."""
    out = [(f"{name}.qweight", "I8" if bits == 8 else "U8", (rows, bytes_per_row), np.asarray(qdata).tobytes()),
           (f"{name}.scales", "F32", (groups, columns), np.asarray(scales, dtype="<f4").tobytes())]
    if zeros is not None:
        out.append((f"{name}.zeros", "U8", (groups, columns), np.asarray(zeros).astype(np.uint8).tobytes()))
    return out
