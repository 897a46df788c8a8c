"""The C ABI library loads and exports every symbol include/*.h declares, and its
argument checks answer like the reference's ``require`` (no device work: these
run without a GPU)."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent


def declared_symbols():
    names = []
    for header in sorted((ROOT / "include").glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        names += re.findall(r"^\s*int32_t\s+(kt_\w+)\s*\(", text, flags=re.M)
    return names


def test_header_declares_the_boundary():
    names = declared_symbols()
    for required in ("kt_quantize", "kt_qmatmul", "kt_qlinear_forward", "kt_qmatmul_transposed",
                     "kt_dequantize_rows", "kt_dequantize_columns", "kt_dev_alloc", "kt_dev_free",
                     "kt_memcpy_h2d", "kt_memcpy_d2h", "kt_stream_create", "kt_stream_sync", "kt_last_error"):
        assert required in names


def test_library_exports_every_declared_symbol():
    import kotensor_amd
    from kotensor_amd import _lib

    lib = _lib.lib()
    for name in declared_symbols():
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    header = (ROOT / "include" / "kotensor_hip.h").read_text()
    declared = int(re.search(r"#define KT_ABI_VERSION (\d+)", header).group(1))
    assert lib.kt_abi_version() == declared == 4
    assert kotensor_amd.LIBRARY_PATH.name == "libkotensor_hip.so"


def test_layout_matches_reference_formulas():
    from kotensor_amd.quantization import layout

    # QuantizationTest.kt:37-74: 100 x 37, int8 g64 and int4 g32
    assert layout(100, 37, 8, 64, False) == (2, 37, 37, 100 * 37 + 2 * 37 * 4)
    assert layout(100, 37, 4, 32, True) == (4, 38, 19, 100 * 19 + 4 * 37 * 4 + 4 * 37)
    # Llama-3-8B FFN, INT4 g64 (the 34,021,376-byte GEMV minus x and y)
    assert layout(4096, 14336, 4, 64, True)[3] == 29360128 + 3670016 + 917504


def test_argument_errors_map_to_illegal_argument():
    from kotensor_amd import _lib, Quantization, IllegalArgumentException

    with pytest.raises(IllegalArgumentException):
        Quantization(3)
    with pytest.raises(IllegalArgumentException):
        Quantization(8, 0)
    assert str(Quantization.INT8) == "int8/g64" and str(Quantization(4, 32)) == "int4/g32"
    lib = _lib.lib()
    fake = ctypes.c_void_p(16)
    assert lib.kt_quantize(fake, 4, 4, 3, 64, fake, fake, None, None) == _lib.KT_ERR_ARGUMENT
    assert "bits must be 4 or 8" in _lib.last_error()
    assert lib.kt_quantize(fake, 4, 4, 8, 0, fake, fake, None, None) == _lib.KT_ERR_ARGUMENT
    assert lib.kt_quantize(fake, 0, 4, 8, 64, fake, fake, None, None) == _lib.KT_ERR_SHAPE
    assert lib.kt_quantize(fake, 4, 4, 4, 64, fake, fake, None, None) == _lib.KT_ERR_ZEROS
    assert "need zero points" in _lib.last_error()
    w = _lib.QWeight(16, 16, None, 8, 8, 4, 64)
    assert lib.kt_qweight_check(ctypes.byref(w)) == _lib.KT_ERR_ZEROS
    w = _lib.QWeight(16, 16, None, 8, 8, 8, 64)
    assert lib.kt_qweight_check(ctypes.byref(w)) == _lib.KT_OK
    assert lib.kt_qmatmul(fake, -1, ctypes.byref(w), fake, 0, ctypes.c_float(1.0), None) == _lib.KT_ERR_ARGUMENT
    assert "Negative row count" in _lib.last_error()
    assert lib.kt_qmatmul(fake, 0, ctypes.byref(w), fake, 0, ctypes.c_float(1.0), None) == _lib.KT_OK
    assert lib.kt_set_kernel_config(6, 0, 0, 0, 0) == _lib.KT_ERR_ARGUMENT
    assert lib.kt_set_kernel_config(0, 5, 0, 0, 0) == _lib.KT_ERR_ARGUMENT
    assert lib.kt_set_kernel_config(0, 0, 0, 3, 0) == _lib.KT_ERR_ARGUMENT
    assert lib.kt_set_kernel_config(0, 0, 0, 0, 3) == _lib.KT_ERR_ARGUMENT
    assert lib.kt_set_kernel_config(0, 0, 0, 0, 0) == _lib.KT_OK
    buf = ctypes.create_string_buffer(8)
    assert lib.kt_last_error(buf, 8) == 0 and len(buf.value) <= 7
    # the column-run copy: size formula, and its checks before any device access
    n = ctypes.c_int64()
    assert lib.kt_qweight_packed_bytes(4096, 14336, 4, 64, ctypes.byref(n)) == _lib.KT_OK
    assert n.value == (14336 // 16) * (4096 // 128) * 1024 + (14336 // 16) * 64 * 80 + 16
    assert lib.kt_qweight_packed_bytes(300, 2100, 8, 32, ctypes.byref(n)) == _lib.KT_OK
    # ceil(2100 / 16) sets, ceil(300 / 128) chunks, 10 groups, the 16-byte trailer
    assert n.value == 132 * 3 * 2048 + 132 * 10 * 80 + 16
    assert lib.kt_qweight_packed_bytes(300, 2100, 5, 32, ctypes.byref(n)) == _lib.KT_ERR_ARGUMENT
    assert lib.kt_qweight_packed_bytes(300, 2100, 8, 0, ctypes.byref(n)) == _lib.KT_ERR_ARGUMENT
    assert lib.kt_qweight_pack(ctypes.byref(w), None, None) == _lib.KT_ERR_ARGUMENT
    assert lib.kt_qweight_pack(ctypes.byref(w), ctypes.c_void_p(8), None) == _lib.KT_ERR_ARGUMENT
    assert "16-byte aligned" in _lib.last_error()
    # the chain of one-row products: its step checks come before any device access
    steps = (_lib.QMatmulStep * 2)()
    assert lib.kt_qmatmul_chain(None, 1, None) == _lib.KT_ERR_ARGUMENT
    assert lib.kt_qmatmul_chain(steps, 0, None) == _lib.KT_ERR_ARGUMENT
    assert lib.kt_qmatmul_chain(steps, 7, None) == _lib.KT_ERR_ARGUMENT
    assert "1 to 6 steps" in _lib.last_error()
    assert lib.kt_qmatmul_chain(steps, 1, None) == _lib.KT_ERR_ARGUMENT  # x, weights, outputs NULL
    outs = (ctypes.c_void_p * 2)(16, 16)
    steps[0].x, steps[0].weights, steps[0].outputs = 16, ctypes.pointer(w), outs
    steps[0].count, steps[0].swiglu_gate = 1, 1
    assert lib.kt_qmatmul_chain(steps, 1, None) == _lib.KT_ERR_ARGUMENT
    assert "SwiGLU gate pair takes 2" in _lib.last_error()


def test_product_does_not_reach_the_oracle():
    """No product source imports, links or names the oracle library."""
    pkg = ROOT / "kotensor_amd"
    for path in list(pkg.rglob("*.py")) + list(pkg.rglob("*.hip")) + list(pkg.rglob("*.h")):
        text = path.read_text()
        assert "kt_oracle" not in text and "import oracle" not in text and "from oracle" not in text, path
    so = (pkg / "libkotensor_hip.so").read_bytes()
    assert b"ko_multiply_quantized" not in so and b"libkt_oracle" not in so
