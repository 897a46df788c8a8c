"""Quantize + pack on the GPU, bit-exact with the oracle (QuantizedTensor.kt:256-324)."""
import json
from pathlib import Path

import numpy as np
import pytest

from gpu_helpers import banner, gpu_quantize, same_bits

pytestmark = pytest.mark.gpu
GOLDEN = Path(__file__).resolve().parent / "golden"


def _kats():
    return json.loads((GOLDEN / "kat_quantize.json").read_text())


def _kat_data(kat):
    return np.array(kat["data_bits"], dtype=np.uint32).view(np.float32).reshape(kat["rows"], kat["columns"])


def _check(kt, oracle_lib, w, bits, g, label):
    banner("quantize", label, w.shape, f"int{bits}/g{g}")
    st, ref = oracle_lib.quantize(w, bits, g)
    if st != 0:
        with pytest.raises(kt.IllegalArgumentException):
            gpu_quantize(kt, w, bits, g)
        return None
    q = gpu_quantize(kt, w, bits, g)
    assert same_bits(q.qdata.view(np.uint8), ref.qdata), label
    assert same_bits(q.scales, ref.scales), label
    if bits == 4:
        assert same_bits(q.zeros, ref.zeros), label
    else:
        assert q.zeros is None
    return q


@pytest.mark.parametrize("kat", _kats(), ids=lambda k: k["name"])
def test_known_answers_on_gpu(kt, oracle_lib, kat):
    w = _kat_data(kat)
    banner("kat", kat["name"])
    k, n = w.shape
    if kat["status"] != 0:
        with pytest.raises(kt.IllegalArgumentException) as err:
            gpu_quantize(kt, w, kat["bits"], kat["group"])
        assert err.value.status == -3
    else:
        q = gpu_quantize(kt, w, kat["bits"], kat["group"])
        want = np.array(kat["qdata"], dtype=np.int64) & 0xFF
        assert q.qdata.view(np.uint8).tolist() == want.tolist()
        assert q.scales.view(np.uint32).tolist() == kat["scales_bits"]
        if kat["bits"] == 4:
            assert q.zeros.tolist() == kat["zeros"]
    # the same columns replicated 8 times run through the vectorised kernels
    wide = np.repeat(w, 8, axis=1)
    _check(kt, oracle_lib, wide, kat["bits"], kat["group"], kat["name"] + "_x8")


SHAPES = [(100, 37), (130, 9001), (300, 2100), (200, 33), (70, 300), (450, 129), (2, 17), (96, 8200),
          (256, 4096), (64, 64), (1, 8), (33, 136)]


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("g", [64, 32, 16, 1, 7, 128, 256, 1000])
def test_random_shapes_bit_exact(kt, oracle_lib, bits, g):
    rng = np.random.default_rng(bits * 1000 + g)
    for k, n in SHAPES:
        w = ((rng.random((k, n), dtype=np.float32) - 0.5) * 0.2).astype(np.float32)
        _check(kt, oracle_lib, w, bits, g, f"rand{k}x{n}")


@pytest.mark.parametrize("bits", [8, 4])
def test_adversarial_values_bit_exact(kt, oracle_lib, bits):
    rng = np.random.default_rng(77 + bits)
    for g in (8, 64):
        k, n = 128, 256
        w = rng.integers(-30, 31, size=(k, n)).astype(np.float32) * np.float32(0.5)
        w[:, 16:32] = np.abs(w[:, 16:32]) + 1
        w[:, 32:48] = -np.abs(w[:, 32:48]) - 1
        w[:, 48:56] = rng.standard_normal((k, 8)).astype(np.float32) * np.float32(1e-40)
        w[:, 56:64] = rng.standard_normal((k, 8)).astype(np.float32) * np.float32(1e37)
        w[:, 64:72] = np.float32(-0.0)
        w[:, 72:80] = 0.0
        w[:, 80:96] = (rng.standard_normal((k, 16)) * 0.02).astype(np.float32)
        _check(kt, oracle_lib, w, bits, g, f"adversarial_g{g}")


def test_saturating_round_bit_exact(kt, oracle_lib):
    """Groups of +-2^-149 values: the scale rounds to 0, the inverse is +inf, x * inverse
    is +-inf and Math.round saturates to Int.MAX_VALUE / MIN_VALUE (INT4: the zero point
    saturates too, and the wrapping add of the zero point decides the nibble)."""
    rng = np.random.default_rng(11)
    tiny = np.float32(1.4e-45)
    for n in (64, 63):  # the vector kernels and the any-shape kernel
        w = (rng.standard_normal((64, n)) * 0.02).astype(np.float32)
        w[:, :24] = np.where(rng.random((64, 24)) < 0.5, -tiny, tiny).astype(np.float32)
        w[:, 24:32] = -tiny
        w[:, 32:40] = tiny  # INT4: min clamps to 0, so zero = round(0 / 0) is NaN: an error
        for bits in (8, 4):
            if bits == 4:
                w[:, 32:40] = -tiny
            for g in (64, 16):
                q = _check(kt, oracle_lib, w, bits, g, f"saturate{n}")
                assert q is not None
                assert np.all(q.scales.reshape(-1, n)[:, :40] == 0.0)


def test_nan_is_rejected_like_round_to_int(kt, oracle_lib):
    w = np.ones((64, 64), dtype=np.float32)
    w[5, 7] = np.nan
    for bits in (4, 8):
        banner("nan", bits)
        with pytest.raises(kt.IllegalArgumentException) as err:
            gpu_quantize(kt, w, bits, 64)
        assert "NaN" in str(err.value)
        # the library keeps working after the error
        ok = np.ones((64, 64), dtype=np.float32)
        _check(kt, oracle_lib, ok, bits, 64, "after_nan")


def test_nan_report_belongs_to_its_call(kt, oracle_lib):
    """The NaN marks are never cleared: each call checks only its own. NaN calls in a row
    all fail, clean calls between and after them all pass, on every kernel path (the
    vector kernels and the generic one)."""
    rng = np.random.default_rng(12)
    for bits, (k, n) in [(4, (64, 64)), (8, (64, 64)), (4, (96, 33)), (8, (70, 9))]:
        banner("nan-sequence", bits, k, n)
        clean = (rng.standard_normal((k, n)) * 0.02).astype(np.float32)
        bad = clean.copy()
        bad[k // 2, n // 3] = np.nan
        for pattern in ("bbcbccb", "cbbbc"):
            for c in pattern:
                if c == "b":
                    with pytest.raises(kt.IllegalArgumentException):
                        gpu_quantize(kt, bad, bits, 32)
                else:
                    _check(kt, oracle_lib, clean, bits, 32, "between_nan")


@pytest.mark.parametrize("shape", [(2048, 2048), (896, 4864), (4864, 896), (2048, 8192), (4096, 14336),
                                   (14336, 4096), (896, 151936)])
@pytest.mark.parametrize("bits", [4, 8])
def test_config_shapes_bit_exact(kt, oracle_lib, shape, bits):
    """Full-size projection weights ~N(0, 0.02), g64 and g32."""
    rng = np.random.default_rng(1)
    k, n = shape
    w = (rng.standard_normal((k, n), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    for g in (64, 32):
        _check(kt, oracle_lib, w, bits, g, f"config{k}x{n}")


def test_llama8b_lm_head_bit_exact(kt, oracle_lib):
    """4096 x 128256 INT4 g64: the largest quantize of the workload set."""
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((4096, 128256), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    _check(kt, oracle_lib, w, 4, 64, "lm_head_8b")
