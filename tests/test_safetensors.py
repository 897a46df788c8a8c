"""The saveQuantized file format (kt_st_*, kotensor_amd.safetensors).

CPU: the library's writer produces exactly the bytes of the oracle's restatement of
SafeTensors.saveEntries (SafeTensors.kt:204-265), the `safetensors` package (an
independent reader) reads them back, the library's reader agrees with both and
answers malformed files with the reference's messages (SafeTensors.kt:37-67), and the
mapFrom size checks (QuantizedTensor.kt:109-125) fire before any device access.
GPU: weights quantized on the device go to a file and back bit for bit, a file
written in the reference layout from oracle-quantized data loads onto the device and
multiplies like the oracle, and a loaded file saved again is identical byte for byte
(MappedModelTest.kt:108-119).
"""
import ctypes
import struct

import numpy as np
import pytest

from conftest import normwise_rel
from oracle import safetensors_ref as ref


def _host_entries(rng):
    f32 = rng.standard_normal((3, 5)).astype(np.float32)
    i8 = rng.integers(-128, 128, size=(7, 4), dtype=np.int8)
    u8 = rng.integers(0, 256, size=(2, 9), dtype=np.uint8)
    scalar = np.array([1.5], dtype=np.float32)
    return [("tok_embeddings.weight", "F32", f32.shape, f32),
            ("block.0.attention.wq.qweight", "I8", i8.shape, i8),
            ('odd "name"\twith\\escapes', "U8", u8.shape, u8),
            ("empty", "F32", (0, 4), np.zeros((0, 4), dtype=np.float32)),
            ("scalar", "F32", (1,), scalar)]


METADATA = {"kotensor.vocabularySize": "32000", "kotensor.normEps": "1.0E-5",
            "kotensor.note": 'quote " backslash \\ newline \n tab \t bell \x07 é'}


def _write_with_library(path, entries, metadata):
    from kotensor_amd import save_entries

    save_entries(path, entries, metadata)


def test_writer_bytes_match_the_reference_layout(tmp_path):
    rng = np.random.default_rng(0)
    entries = _host_entries(rng)
    path = tmp_path / "a.safetensors"
    _write_with_library(path, entries, METADATA)
    expected = ref.write_entries([(n, d, s, np.ascontiguousarray(a).tobytes()) for n, d, s, a in entries], METADATA)
    assert path.read_bytes() == expected
    # header size multiple of 8, padded with spaces
    (size,) = struct.unpack_from("<q", expected, 0)
    assert size % 8 == 0


def test_independent_reader_reads_library_files(tmp_path):
    from safetensors import safe_open

    rng = np.random.default_rng(1)
    entries = _host_entries(rng)
    path = tmp_path / "b.safetensors"
    _write_with_library(path, entries, METADATA)
    with safe_open(str(path), framework="numpy") as f:
        assert f.metadata() == METADATA
        for name, _dtype, _shape, arr in entries:
            np.testing.assert_array_equal(f.get_tensor(name), arr)


def test_library_reader_agrees_with_the_oracle(tmp_path):
    from kotensor_amd import SafeTensorsFile

    rng = np.random.default_rng(2)
    entries = _host_entries(rng)
    raw = ref.write_entries([(n, d, s, np.ascontiguousarray(a).tobytes()) for n, d, s, a in entries], METADATA)
    path = tmp_path / "c.safetensors"
    path.write_bytes(raw)
    want_entries, want_meta = ref.read_header(raw)
    with SafeTensorsFile(path) as f:
        assert f.names == [n for n, *_ in entries]  # header order
        assert f.metadata == want_meta == METADATA
        for name, dtype, shape, arr in entries:
            e = f.entry(name)
            wd, ws, start, end = want_entries[name]
            assert (e.dtype, e.shape, e.byte_offset, e.byte_length) == (wd, tuple(ws), start, end - start)
            assert f.read_raw(name).tobytes() == np.ascontiguousarray(arr).tobytes()
        np.testing.assert_array_equal(f.load("tok_embeddings.weight"), entries[0][3])
        np.testing.assert_array_equal(f.load("block.0.attention.wq.qweight"), entries[1][3].astype(np.float32))
        assert "missing" not in f and "scalar" in f


def _bad_file(tmp_path, name, header: bytes, data: bytes = b"", size=None):
    size = len(header) if size is None else size
    path = tmp_path / name
    path.write_bytes(struct.pack("<q", size) + header + data)
    return path


def test_reader_rejects_malformed_files_like_the_reference(tmp_path):
    from kotensor_amd import IllegalArgumentException, SafeTensorsFile

    cases = [
        (_bad_file(tmp_path, "zero.st", b"{}", size=0), "Invalid safetensors header size 0"),
        (_bad_file(tmp_path, "big.st", b"{}", size=(100 << 20) + 1), "Invalid safetensors header size"),
        (_bad_file(tmp_path, "list.st", b"[1,2]   "), "is not a JSON object"),
        (_bad_file(tmp_path, "nodtype.st", b'{"a":{"shape":[1],"data_offsets":[0,4]}}', b"\0" * 4), "Tensor a has no dtype"),
        (_bad_file(tmp_path, "nooff.st", b'{"a":{"dtype":"F32","shape":[1]}}'), "Tensor a has no data_offsets"),
        (_bad_file(tmp_path, "range.st", b'{"a":{"dtype":"F32","shape":[4],"data_offsets":[0,16]}}', b"\0" * 8),
         "Tensor a data range [0, 16) exceeds file"),
        # data_start + end would wrap past INT64_MAX into a small number: still rejected
        (_bad_file(tmp_path, "wrap.st", b'{"a":{"dtype":"F32","shape":[1],'
                   b'"data_offsets":[9223372036854775803,9223372036854775807]}}', b"\0" * 4),
         "Tensor a data range [9223372036854775803, 9223372036854775807) exceeds file"),
        (_bad_file(tmp_path, "neg.st", b'{"a":{"dtype":"F32","shape":[1],"data_offsets":[-4,0]}}', b"\0" * 4),
         "Tensor a data range [-4, 0) exceeds file"),
        (_bad_file(tmp_path, "huge.st", b'{"a":{"dtype":"F32","shape":[1],"data_offsets":[0,99999999999999999999]}}',
                   b"\0" * 4), "Tensor a has no data_offsets"),
    ]
    for path, message in cases:
        with pytest.raises(IllegalArgumentException) as err:
            SafeTensorsFile(path)
        assert message in str(err.value), (path.name, str(err.value))
    with pytest.raises(IllegalArgumentException):
        SafeTensorsFile(tmp_path / "does-not-exist.st")
    ok = _bad_file(tmp_path, "ok.st", b'{"__metadata__":{"k":"v"},"skip":1,"a":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}}',
                   b"\0" * 4)
    with SafeTensorsFile(ok) as f:
        assert f.names == ["a"]  # non-object values are skipped, as the reference does
        with pytest.raises(IllegalArgumentException, match="No tensor named 'b'"):
            f.entry("b")
        with pytest.raises(IllegalArgumentException, match="No tensor named 'b'"):
            f.map("b")


def test_mapfrom_size_checks_before_device_access(tmp_path):
    """QuantizedTensor.mapFrom's checks (QuantizedTensor.kt:110-117) run on the host: a
    mismatched file is rejected without touching the (fake) device pointers."""
    from kotensor_amd import IllegalArgumentException, SafeTensorsFile, _lib

    rows, columns, g = 8, 6, 4  # INT4: bytesPerRow 3, groups 2
    good_q = np.zeros((rows, 3), dtype=np.uint8)
    scales = np.ones((2, columns), dtype=np.float32)
    zeros = np.zeros((2, columns), dtype=np.uint8)
    variants = {
        "qweight": ([("w.qweight", "U8", (rows, 2), np.zeros((rows, 2), np.uint8).tobytes()),
                     ("w.scales", "F32", (2, columns), scales.tobytes()), ("w.zeros", "U8", (2, columns), zeros.tobytes())],
                    "w.qweight has 16 bytes, expected 24"),
        "scales": ([("w.qweight", "U8", (rows, 3), good_q.tobytes()),
                    ("w.scales", "F16", (2, columns), np.ones((2, columns), np.float16).tobytes()),
                    ("w.zeros", "U8", (2, columns), zeros.tobytes())],
                   "w.scales is F16 with 24 bytes, expected F32 with 48"),
        "zeros": ([("w.qweight", "U8", (rows, 3), good_q.tobytes()), ("w.scales", "F32", (2, columns), scales.tobytes()),
                   ("w.zeros", "U8", (1, columns), np.zeros((1, columns), np.uint8).tobytes())],
                  "w.zeros has 6 bytes, expected 12"),
        "missing": ([("w.qweight", "U8", (rows, 3), good_q.tobytes()), ("w.scales", "F32", (2, columns), scales.tobytes())],
                    "No tensor named 'w.zeros'"),
    }
    fake = 0x1000  # never dereferenced: the checks fail first
    for key, (entries, message) in variants.items():
        path = tmp_path / f"{key}.st"
        path.write_bytes(ref.write_entries(entries))
        with SafeTensorsFile(path) as f:
            w = _lib.QWeight(fake, fake, fake, rows, columns, 4, g)
            with pytest.raises(IllegalArgumentException) as err:
                _lib.call("kt_st_load_qweight", f._h, b"w", ctypes.byref(w), None)
            assert message in str(err.value), (key, str(err.value))


# ---- on the device -------------------------------------------------------------------


@pytest.mark.gpu
@pytest.mark.parametrize("bits,g", [(4, 64), (8, 32), (4, 32)])
def test_device_weights_round_trip_through_a_file(kt, oracle_lib, tmp_path, bits, g):
    rng = np.random.default_rng(10 + bits)
    rows, columns = 256, 200
    data = (rng.standard_normal((rows, columns)) * 0.02).astype(np.float32)
    q = kt.Quantization(bits, g)
    w = kt.QuantizedTensor.quantize(data, rows, columns, q)
    params = {"norm.weight": rng.standard_normal(64).astype(np.float32)}
    meta = {"kotensor.dimension": "64", "kotensor.quantization.bits": str(bits),
            "kotensor.quantization.groupSize": str(g)}
    path = tmp_path / "m.safetensors"
    kt.save_quantized(path, params, {"block.0.ffn.wDown": w}, meta)
    meta2, params2, quantized2 = kt.load_quantized(path)
    assert meta2 == meta
    np.testing.assert_array_equal(params2["norm.weight"], params["norm.weight"])
    w2 = quantized2["block.0.ffn.wDown"]
    assert (w2.rows, w2.columns, w2.bits, w2.group_size) == (rows, columns, bits, g)
    np.testing.assert_array_equal(w2.qdata, w.qdata)
    np.testing.assert_array_equal(w2.scales, w.scales)
    if bits == 4:
        np.testing.assert_array_equal(w2.zeros, w.zeros)
    else:
        assert w2.zeros is None
    # the loaded weight multiplies exactly like the original
    x = rng.standard_normal((1, rows)).astype(np.float32)
    y1 = kt.DeviceTensor.from_numpy(x).matmul_dequant(w).numpy()
    y2 = kt.DeviceTensor.from_numpy(x).matmul_dequant(w2).numpy()
    np.testing.assert_array_equal(y1, y2)
    # saved again: identical file
    path2 = tmp_path / "m2.safetensors"
    kt.save_quantized(path2, params2, quantized2, meta2)
    assert path2.read_bytes() == path.read_bytes()


@pytest.mark.gpu
def test_reference_layout_file_loads_and_matches_the_oracle(kt, oracle_lib, tmp_path):
    rng = np.random.default_rng(21)
    rows, columns, bits, g = 320, 96, 4, 64
    data = (rng.standard_normal((rows, columns)) * 0.05).astype(np.float32)
    status, qw = oracle_lib.quantize(data, bits, g)
    assert status == 0
    entries = ref.quantized_entries("lm_head", bits, rows, qw.bytes_per_row, qw.groups, columns, qw.qdata, qw.scales,
                                    qw.zeros)
    meta = {"kotensor.quantization.bits": "4", "kotensor.quantization.groupSize": "64", "kotensor.tiedEmbedding": "true"}
    path = tmp_path / "ref.safetensors"
    path.write_bytes(ref.write_entries(entries, meta))
    meta2, _, quantized = kt.load_quantized(path)
    assert meta2["kotensor.tiedEmbedding"] == "true"
    w = quantized["lm_head"]
    np.testing.assert_array_equal(w.qdata.view(np.uint8), qw.qdata.reshape(-1))
    x = rng.standard_normal((3, rows)).astype(np.float32)
    got = kt.DeviceTensor.from_numpy(x).matmul_dequant(w).numpy()
    want = oracle_lib.multiply_quantized(x, qw, 3)
    assert normwise_rel(got, want) <= 2e-3
