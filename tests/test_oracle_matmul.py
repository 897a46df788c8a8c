"""Pins the oracle's dequantizing matmul and its transposed product (CPU only).

  * fp64 brute force on weights decoded by the independent numpy decoder, on the
    shapes and schemes of QuantizationTest.kt:76-108 and DecodeKernelTest.kt:47-90,
    with the reference's tolerances (1e-4 forward, 1e-3 backward);
  * the reference's bit-for-bit invariants: the M == 1 result does not depend on
    the thread count (DecodeKernelTest.kt:47-77,92-109, QuantizationTest.kt:110-134);
  * batched rows equal the single-row kernel within 1e-4 (QuantizationTest.kt:126-130);
  * the M == 1 unit decomposition of MatMul.kt:494-512 on hand-computed shapes.
"""
import numpy as np
import pytest

import spec_numpy

SCHEMES = [(8, 64), (4, 64), (4, 32), (8, 1000)]


def _decoded(q):
    return spec_numpy.decode(q.qdata, q.scales, q.zeros, q.rows, q.columns, q.bits, q.group_size).astype(np.float64)


@pytest.mark.parametrize("m,k,n", [(1, 70, 300), (1, 64, 64), (5, 130, 577), (40, 96, 33), (1, 256, 1537)])
def test_matmul_matches_fp64_brute_force(oracle_lib, m, k, n):
    rng = np.random.default_rng(2)
    a = (rng.random((m, k), dtype=np.float32) - 0.5).astype(np.float32)
    w = ((rng.random((k, n), dtype=np.float32) - 0.5) * 0.2).astype(np.float32)
    for bits, g in SCHEMES:
        st, q = oracle_lib.quantize(w, bits, g)
        assert st == 0
        expected = a.astype(np.float64) @ _decoded(q)
        actual = oracle_lib.multiply_quantized(a, q, m)
        assert np.abs(actual - expected).max() < 1e-4, (bits, g)
        acc = oracle_lib.multiply_quantized(a, q, m, c=np.ones((m, n), np.float32), accumulate=True, alpha=0.5)
        assert np.abs(acc - (1.0 + 0.5 * expected)).max() < 1e-4
        dy = (rng.random((m, n), dtype=np.float32) - 0.5).astype(np.float32)
        # backward dequantizes rows like dequantizeRow: 8-bit ignores zero points
        dx = oracle_lib.multiply_by_quantized_transposed(dy, q, m)
        assert np.abs(dx - dy.astype(np.float64) @ _decoded(q).T).max() < 1e-3


def test_matmul_catches_a_planted_mistake(oracle_lib):
    """The brute-force check is sharp enough: dropping the zero-point term fails it."""
    rng = np.random.default_rng(3)
    a = (rng.random((1, 130), dtype=np.float32) - 0.5).astype(np.float32)
    w = ((rng.random((130, 577), dtype=np.float32) - 0.5) * 0.2).astype(np.float32)
    st, q = oracle_lib.quantize(w, 4, 64)
    truth = a.astype(np.float64) @ _decoded(q)
    bad = q.qdata.copy()
    q_no_zero = oracle_lib.Quantized(bad, q.scales, np.zeros_like(q.zeros), 130, 577, 4, 64)
    wrong = oracle_lib.multiply_quantized(a, q_no_zero, 1)
    assert np.abs(wrong - truth).max() > 1e-2
    transposed = oracle_lib.Quantized(q.qdata, q.scales, q.zeros, 130, 577, 4, 64)
    assert np.abs(oracle_lib.multiply_quantized(a, transposed, 1) - truth).max() < 1e-4


@pytest.mark.parametrize("k,n", [(130, 9001), (300, 2100), (200, 33), (70, 300), (450, 129), (2, 17)])
def test_row_kernel_is_thread_count_invariant(oracle_lib, k, n):
    rng = np.random.default_rng(8)
    w = ((rng.random((k, n), dtype=np.float32) - 0.5) * 0.2).astype(np.float32)
    a = (rng.random((1, k), dtype=np.float32) - 0.5).astype(np.float32)
    for bits, g in [(4, 64), (4, 32), (8, 64)]:
        st, q = oracle_lib.quantize(w, bits, g)
        reference = a.astype(np.float64) @ _decoded(q)
        first = oracle_lib.multiply_quantized(a, q, 1, threads=1)
        assert np.abs(first - reference).max() < 1e-4
        for threads in (3, 4):
            assert np.array_equal(first, oracle_lib.multiply_quantized(a, q, 1, threads=threads))


def test_row_kernel_accumulates_with_alpha(oracle_lib):
    """DecodeKernelTest.kt:79-90: the column-split path (N >= 8192) with alpha -0.5."""
    rng = np.random.default_rng(9)
    k, n = 96, 8200
    st, q = oracle_lib.quantize((rng.random((k, n), dtype=np.float32) - 0.5).astype(np.float32), 4, 64)
    a = (rng.random((1, k), dtype=np.float32) - 0.5).astype(np.float32)
    plain = oracle_lib.multiply_quantized(a, q, 1)
    acc = oracle_lib.multiply_quantized(a, q, 1, c=np.full((1, n), 2.0, np.float32), accumulate=True, alpha=-0.5)
    assert np.abs(acc - (2.0 - 0.5 * plain)).max() < 1e-4


def test_batched_rows_match_row_kernel(oracle_lib):
    """QuantizationTest.kt:110-134."""
    rng = np.random.default_rng(4)
    k, n = 300, 2100
    a = (rng.random((1, k), dtype=np.float32) - 0.5).astype(np.float32)
    st, q = oracle_lib.quantize((rng.random((k, n), dtype=np.float32) - 0.5).astype(np.float32), 4, 64)
    serial = oracle_lib.multiply_quantized(a, q, 1, threads=1)
    assert np.array_equal(serial, oracle_lib.multiply_quantized(a, q, 1, threads=8))
    batched = oracle_lib.multiply_quantized(np.tile(a, (3, 1)), q, 3, threads=4)
    for r in range(3):
        assert np.abs(batched[r] - serial[0]).max() < 1e-4


def test_unit_decomposition_known_answers(oracle_lib):
    """MatMul.kt:494-512 worked by hand.
    K = N = 2048, INT8 g64: targetUnits = min(2048*2048/65536, 48) = 48; groups = 32 ->
    groupsPerUnit = 1 -> rowsPerUnit = 64, rowUnits = 32; wantedColumnUnits =
    ceil(48*64/2048) = 2; columnUnits = 2 (<= 2048/128); blockBytes = 1024, blocks = 2.
    K = 896, N = 151936, INT4 g64 (column split): rowsPerUnit = K, targetUnits = 48,
    columnUnits = 48, rowBytes = 75968, blockBytes = roundup64(ceil(75968/48)=1583) = 1600,
    blocks = ceil(75968/1600) = 48."""
    def units(k, n, bits, g):
        bpr = oracle_lib.bytes_per_row(n, bits)
        q = oracle_lib.Quantized(np.zeros(k * bpr, np.uint8), np.ones(oracle_lib.groups(k, g) * n, np.float32),
                                 np.zeros(oracle_lib.groups(k, g) * n, np.int8) if bits == 4 else None, k, n, bits, g)
        return q.row_units()

    assert units(2048, 2048, 8, 64) == [48, 64, 32, 2, 1024, 2]
    assert units(896, 151936, 4, 64) == [48, 896, 1, 48, 1600, 48]
    # K = 4096, N = 4096, INT4 g64: groups 64 -> groupsPerUnit 2 -> rowsPerUnit 128, rowUnits 32;
    # wanted = ceil(48*128/4096) = 2; rowBytes 2048 -> blockBytes 1024, blocks 2.
    assert units(4096, 4096, 4, 64) == [48, 128, 32, 2, 1024, 2]
    # tiny: K = 2, N = 17 INT8: targetUnits 1, groups 1 -> rowsPerUnit = min(2, 64) = 2, 1 row unit,
    # columnUnits clamp(1, 1, max(1, 17/128 = 0)) = 1, blockBytes = min(17, 64) = 17, blocks 1.
    assert units(2, 17, 8, 64) == [1, 2, 1, 1, 17, 1]
