"""Pins the oracle's quantize, packing and dequant accessors (CPU only).

Checks, each chosen so a plausible mistake fails one of them:
  * hand-derived known answers (tests/golden/kat_quantize.json): ties toward +inf
    (half-away or half-even fail), 0.49999997f (floor(x + 0.5f) fails), split-half
    packing with a pad nibble (adjacent-pair packing or swapped nibbles fail),
    zero-point clamps, maxAbs = 0, subnormal scales, Kotlin's wrapping Int
    addition, inf/NaN errors, reciprocal-multiply for q and true division for the
    zero point (the searched cases fail the other operation);
  * the structural known answers of QuantizationTest.kt:37-74;
  * an independent numpy restatement (tests/spec_numpy.py) on random and
    adversarial data, byte for byte.
"""
import json
from pathlib import Path

import numpy as np
import pytest

import spec_numpy

GOLDEN = Path(__file__).resolve().parent / "golden"


def kats():
    return json.loads((GOLDEN / "kat_quantize.json").read_text())


def _data(kat):
    bits = np.array(kat["data_bits"], dtype=np.uint32)
    return bits.view(np.float32).reshape(kat["rows"], kat["columns"])


@pytest.mark.parametrize("kat", kats(), ids=lambda k: k["name"])
def test_oracle_matches_known_answers(oracle_lib, kat):
    st, q = oracle_lib.quantize(_data(kat), kat["bits"], kat["group"])
    assert st == kat["status"]
    if kat["status"] != 0:
        return
    if kat["bits"] == 8:
        assert q.qdata.view(np.int8).tolist() == kat["qdata"]
        assert q.zeros is None
    else:
        assert q.qdata.tolist() == kat["qdata"]
        assert q.zeros.tolist() == kat["zeros"]
    assert q.scales.view(np.uint32).tolist() == kat["scales_bits"]


@pytest.mark.parametrize("kat", kats(), ids=lambda k: k["name"])
def test_numpy_restatement_matches_known_answers(kat):
    """The cross-check implementation is itself held to the same answers."""
    data = _data(kat)
    if kat["status"] != 0:
        with pytest.raises(spec_numpy.RoundNaN):
            spec_numpy.quantize(data, kat["bits"], kat["group"])
        return
    qd, s, z = spec_numpy.quantize(data, kat["bits"], kat["group"])
    expect = np.array(kat["qdata"], dtype=np.int64) & 0xFF
    assert qd.tolist() == expect.tolist()
    assert s.view(np.uint32).tolist() == kat["scales_bits"]


def test_java_round_contract(oracle_lib):
    cases = {0.5: 1, -0.5: 0, 1.5: 2, -1.5: -1, 2.5: 3, -2.5: -2, 0.49999997: 0, -0.49999997: 0,
             -1e-30: 0, 1e-30: 0, 8388607.5: 8388608, -8388607.5: -8388607, 3e9: 2**31 - 1,
             -3e9: -2**31, float("inf"): 2**31 - 1, float("-inf"): -2**31, 126.99999: 127}
    for x, want in cases.items():
        got, nan = oracle_lib.java_round(x)
        assert not nan
        assert got == want, x
    assert oracle_lib.java_round(float("nan"))[1]


def test_structural_known_answers(oracle_lib):
    """QuantizationTest.kt:37-74 on 100 x 37 data in (-0.3, 0.3)."""
    rng = np.random.default_rng(1)
    rows, columns = 100, 37
    w = ((rng.random((rows, columns), dtype=np.float32) * 2 - 1) * 0.3).astype(np.float32)
    st, int8 = oracle_lib.quantize(w, 8, 64)
    assert st == 0
    assert int8.groups == 2 and int8.zeros is None and int8.qdata.size == rows * columns
    assert np.abs(w - int8.dequantize()).max() <= 0.3 / 127 + 1e-6
    st, int4 = oracle_lib.quantize(w, 4, 32)
    assert st == 0
    assert int4.groups == 4 and int4.bytes_per_row == 19 and int4.qdata.size == rows * 19
    assert int4.zeros.size == 4 * columns
    assert (columns + columns % 2) == 38  # storedColumns
    assert np.abs(w - int4.dequantize()).max() <= 0.6 / 15 / 2 + 1e-6
    deq = int4.dequantize()
    for r in range(0, rows, 7):
        for c in range(columns):
            assert 0 <= int4.raw_value(r, c) <= 15
            assert int4.value(r, c) == deq[r, c]
    zeros = np.zeros((rows, columns), dtype=np.float32)
    for bits in (4, 8):
        st, qz = oracle_lib.quantize(zeros, bits, 64)
        assert st == 0 and np.abs(qz.dequantize()).max() == 0.0
    # sizeInBytes, QuantizedTensor.kt:97-98
    assert rows * columns + 2 * columns * 4 == int8.qdata.size + int8.scales.size * 4
    assert rows * 19 + 4 * columns * 4 + 4 * columns == int4.qdata.size + int4.scales.size * 4 + int4.zeros.size


SHAPES = [(100, 37), (130, 129), (200, 33), (70, 300), (450, 129), (2, 17), (64, 64), (256, 1537), (1, 5), (7, 8)]
GROUPS = [64, 32, 16, 1, 7, 1000]


@pytest.mark.parametrize("bits", [8, 4])
@pytest.mark.parametrize("shape", SHAPES)
def test_oracle_matches_numpy_restatement(oracle_lib, bits, shape):
    rng = np.random.default_rng(hash((bits,) + shape) % 2**32)
    k, n = shape
    for g in GROUPS:
        w = ((rng.random((k, n), dtype=np.float32) - 0.5) * 0.2).astype(np.float32)
        st, q = oracle_lib.quantize(w, bits, g)
        assert st == 0
        qd, s, z = spec_numpy.quantize(w, bits, g)
        assert np.array_equal(q.qdata, qd), (shape, g)
        assert np.array_equal(q.scales.view(np.uint32), s.view(np.uint32)), (shape, g)
        if bits == 4:
            assert np.array_equal(q.zeros, z), (shape, g)
        deq = spec_numpy.decode(q.qdata, q.scales, q.zeros, k, n, bits, g)
        for r in range(0, k, max(1, k // 5)):
            assert np.array_equal(q.dequantize_row(r), deq[r])
        for c in range(0, n, max(1, n // 5)):
            assert np.array_equal(q.dequantize_column(c), deq[:, c])


@pytest.mark.parametrize("bits", [8, 4])
def test_oracle_adversarial_values_match_numpy(oracle_lib, bits):
    """Exact ties, huge and subnormal magnitudes, signed zeros, one-signed groups."""
    rng = np.random.default_rng(7 + bits)
    k, n, g = 64, 96, 8
    w = rng.integers(-30, 31, size=(k, n)).astype(np.float32) * np.float32(0.5)  # many exact .5 ties
    w[:, 10:20] = np.abs(w[:, 10:20]) + 1
    w[:, 20:30] = -np.abs(w[:, 20:30]) - 1
    w[:, 30:35] = rng.standard_normal((k, 5)).astype(np.float32) * np.float32(1e-40)
    w[:, 35:40] = rng.standard_normal((k, 5)).astype(np.float32) * np.float32(1e37)
    w[:, 40:44] = np.float32(-0.0)
    w[:, 44:48] = 0.0
    st, q = oracle_lib.quantize(w, bits, g)
    try:
        qd, s, z = spec_numpy.quantize(w, bits, g)
        expect = 0
    except spec_numpy.RoundNaN:
        expect = -3
    assert st == expect
    if st == 0:
        assert np.array_equal(q.qdata, qd)
        assert np.array_equal(q.scales.view(np.uint32), s.view(np.uint32))
        if bits == 4:
            assert np.array_equal(q.zeros, z)


def test_golden_fixtures_reproduce(oracle_lib):
    """The committed regression vectors still come out of the oracle bit for bit."""
    data = np.load(GOLDEN / "fixtures.npz")
    names = sorted({k.split(".")[0] for k in data.files})
    assert names
    for name in names:
        k, n, bits, g = (int(v) for v in data[f"{name}.meta"])
        st, q = oracle_lib.quantize(data[f"{name}.data"], bits, g)
        assert st == 0
        assert np.array_equal(q.qdata, data[f"{name}.qdata"]), name
        assert np.array_equal(q.scales.view(np.uint32), data[f"{name}.scales"].view(np.uint32)), name
        if bits == 4:
            assert np.array_equal(q.zeros, data[f"{name}.zeros"]), name
        x = data[f"{name}.x"]
        assert np.array_equal(oracle_lib.multiply_quantized(x, q, 3), data[f"{name}.y3"]), name
        assert np.array_equal(oracle_lib.multiply_quantized(x[:1], q, 1), data[f"{name}.y1"]), name


def test_column_run_spec_matches_its_definition():
    """tests/spec_numpy.pack_column_runs (reshapes) against the layout's per-byte
    definition, on ragged INT4/INT8 shapes with random bytes."""
    from spec_numpy import pack_column_runs
    rng = np.random.default_rng(0)
    for K, N, bits in [(300, 2100, 4), (300, 2100, 8), (128, 16, 8), (200, 33, 4), (70, 9, 4)]:
        bpr = (N + N % 2) // 2 if bits == 4 else N
        q = rng.integers(0, 256, size=K * bpr, dtype=np.uint8)
        Q = q.reshape(K, bpr)
        if bits == 4 and N % 2:
            Q[:, -1] &= 0x0F  # the pad nibble is 0

        def val(k, c):
            if k >= K or c >= N:
                return 0
            if bits == 8:
                return int(Q[k, c])
            return int(Q[k, c] & 15) if c < bpr else int(Q[k, c - bpr] >> 4)

        P = pack_column_runs(q, K, N, bits)
        sets, chunks, BB = -(-N // 16), -(-K // 128), 1024 if bits == 4 else 2048
        assert P.size == sets * chunks * BB
        for _ in range(2000):
            s, c, lane = rng.integers(sets), rng.integers(chunks), rng.integers(64)
            col, run = 16 * s + (lane & 15), 128 * c + 32 * (lane >> 4)
            if bits == 8:
                h, b = rng.integers(2), rng.integers(16)
                assert P[(s * chunks + c) * BB + h * 1024 + 16 * lane + b] == val(run + 16 * h + b, col)
            else:
                d, t = rng.integers(4), rng.integers(4)
                k = run + 16 * (d >> 1) + 8 * (d & 1) + t
                assert P[(s * chunks + c) * BB + 16 * lane + 4 * d + t] == val(k, col) | (val(k + 4, col) << 4)
        # the scale and zero-point rows after the blocks: row (set, group) holds the 16
        # columns of the set, fp32 scales first, then the zero points' bytes
        for g in (32, 64, 96):
            G = -(-K // g)
            sc = rng.standard_normal(G * N).astype(np.float32)
            zs = rng.integers(0, 16, size=G * N, dtype=np.uint8)
            P = pack_column_runs(q, K, N, bits, sc, zs, g)
            base = sets * chunks * BB
            assert P.size == base + sets * G * 80 + 16
            srows = P[base:base + sets * G * 64].view(np.float32)
            zrows = P[base + sets * G * 64:base + sets * G * 80]
            # the trailer: the largest |scale| over every scale (columns past N hold 0)
            trailer = P[base + sets * G * 80:].view(np.float32)
            assert trailer[0] == np.abs(sc).max() and not trailer[1:].any()
            for _ in range(500):
                s, grp, n = rng.integers(sets), rng.integers(G), rng.integers(16)
                col = 16 * s + n
                want_s = sc[grp * N + col] if col < N else 0.0
                want_z = zs[grp * N + col] if col < N else 0
                assert srows[(s * G + grp) * 16 + n] == want_s
                assert zrows[(s * G + grp) * 16 + n] == want_z
