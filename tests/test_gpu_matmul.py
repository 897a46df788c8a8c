"""Dequantizing matmul on the GPU against the oracle's MatMul.multiplyQuantized.

Criterion (fp32 in/out): normwise relative error ||gpu - oracle|| / ||oracle|| <= 2e-3.
The M == 1 kernel accumulates in fp32 and lands near 1e-7; the MFMA kernel rounds
both operands to fp16 (relative 2^-11) and lands near 3e-4.
"""
import numpy as np
import pytest

from conftest import normwise_rel
from gpu_helpers import banner, gpu_matmul, raw_ptr, same_bits, upload_quantized

pytestmark = pytest.mark.gpu
TOL = 2e-3
SCHEMES = [(8, 64), (4, 64), (4, 32), (8, 1000)]


def _weights(oracle_lib, k, n, bits, g, seed, std=None):
    rng = np.random.default_rng(seed)
    if std is None:
        w = ((rng.random((k, n), dtype=np.float32) - 0.5) * 0.2).astype(np.float32)
    else:
        w = (rng.standard_normal((k, n), dtype=np.float32) * np.float32(std)).astype(np.float32)
    st, q = oracle_lib.quantize(w, bits, g)
    assert st == 0
    return q


def _compare(kt, oracle_lib, q, x, label, rows=None, c0=None, accumulate=False, alpha=1.0, tol=TOL):
    m = x.shape[0]
    banner("matmul", label, f"M={m}", f"K={q.rows}", f"N={q.columns}", f"int{q.bits}/g{q.group_size}")
    qt = upload_quantized(kt, q)
    got = gpu_matmul(kt, x, qt, m, c0=c0, accumulate=accumulate, alpha=alpha)
    idx = np.arange(m) if rows is None else np.asarray(rows)
    ref_c0 = None if c0 is None else c0[idx]
    want = oracle_lib.multiply_quantized(x[idx], q, len(idx), c=ref_c0, accumulate=accumulate, alpha=alpha,
                                         threads=16)
    err = normwise_rel(got[idx], want)
    print(f"  normwise={err:.3e}", flush=True)
    assert err <= tol, (label, err)
    return got, want


@pytest.mark.parametrize("m,k,n", [(1, 70, 300), (1, 64, 64), (5, 130, 577), (40, 96, 33), (1, 256, 1537),
                                   (3, 256, 1536), (17, 640, 1024)])
def test_reference_shapes(kt, oracle_lib, m, k, n):
    """QuantizationTest.kt:76-108 shapes (plus aligned ones that take the fast kernels)."""
    rng = np.random.default_rng(2)
    x = (rng.random((m, k), dtype=np.float32) - 0.5).astype(np.float32)
    for bits, g in SCHEMES:
        q = _weights(oracle_lib, k, n, bits, g, 10 + bits + g)
        got, want = _compare(kt, oracle_lib, q, x, "ref")
        assert np.abs(got - want).max() < 1e-3
        ones = np.ones((m, n), dtype=np.float32)
        _compare(kt, oracle_lib, q, x, "ref-acc", c0=ones, accumulate=True, alpha=0.5)


@pytest.mark.parametrize("k,n", [(130, 9001), (300, 2100), (200, 33), (70, 300), (450, 129), (2, 17),
                                 (256, 4096), (96, 8200)])
def test_decode_kernel_shapes(kt, oracle_lib, k, n):
    """DecodeKernelTest.kt:47-90 shapes at M == 1, with alpha -0.5 accumulation."""
    rng = np.random.default_rng(8)
    x = (rng.random((1, k), dtype=np.float32) - 0.5).astype(np.float32)
    for bits, g in [(4, 64), (4, 32), (8, 64)]:
        q = _weights(oracle_lib, k, n, bits, g, k + n + bits)
        _compare(kt, oracle_lib, q, x, "decode")
        c0 = np.full((1, n), 2.0, dtype=np.float32)
        _compare(kt, oracle_lib, q, x, "decode-acc", c0=c0, accumulate=True, alpha=-0.5)


QWEN = [(896, 896), (896, 128), (896, 4864), (4864, 896), (896, 151936)]


@pytest.mark.parametrize("k,n", QWEN)
@pytest.mark.parametrize("g", [64, 32])
def test_qwen_int4_gemv(kt, oracle_lib, k, n, g):
    """INT4 M == 1 on the Qwen2-0.5B projection shapes, x ~ N(0,1), W ~ N(0, 0.02)."""
    rng = np.random.default_rng(0)
    x = rng.standard_normal((1, k), dtype=np.float32)
    q = _weights(oracle_lib, k, n, 4, g, 1, std=0.02)
    _compare(kt, oracle_lib, q, x, "qwen")


@pytest.mark.parametrize("g", [64, 32])
def test_int8_gemv_2048(kt, oracle_lib, g):
    rng = np.random.default_rng(0)
    x = rng.standard_normal((1, 2048), dtype=np.float32)
    q = _weights(oracle_lib, 2048, 2048, 8, g, 1, std=0.02)
    _compare(kt, oracle_lib, q, x, "int8-gemv")


LLAMA1B = [(2048, 2048), (2048, 512), (2048, 8192), (8192, 2048)]


def tile_rows(m: int, rng, every: int = 512) -> np.ndarray:
    """Rows the oracle checks: all of them up to `every` rows, above that the first and
    last row and one random row of every 128-row tile of the GEMM (so no tile, and no
    position of the workgroup-to-tile mapping, goes unchecked)."""
    if m <= every:
        return np.arange(m)
    tiles = np.arange(0, m, 128)
    picks = [tiles, np.minimum(tiles + 127, m - 1), np.minimum(tiles + rng.integers(1, 127, tiles.size), m - 1)]
    return np.unique(np.concatenate(picks))


@pytest.mark.parametrize("k,n", LLAMA1B)
@pytest.mark.parametrize("m", [1, 16, 128, 512, 2048])
def test_int8_prefill_sweep(kt, oracle_lib, m, k, n):
    """INT8 g64 on Llama-3.2-1B-like shapes; every 128-row tile is checked."""
    rng = np.random.default_rng(m + k + n)
    x = rng.standard_normal((m, k), dtype=np.float32)
    q = _weights(oracle_lib, k, n, 8, 64, 1, std=0.02)
    _compare(kt, oracle_lib, q, x, "prefill", rows=tile_rows(m, rng))


@pytest.mark.parametrize("k,n", LLAMA1B)
@pytest.mark.parametrize("m", [17, 128, 512, 2048])
def test_int8_g32_gemm_every_tile(kt, oracle_lib, m, k, n):
    """INT8 g32 -- the configuration the prefill GEMM figures are measured on -- through
    the GEMM (M >= 17): with g = 32 every 64-deep K step spans two groups. All rows up
    to M = 512, rows from every 128-row tile at M = 2048."""
    rng = np.random.default_rng(7 * m + k + n)
    x = rng.standard_normal((m, k), dtype=np.float32)
    q = _weights(oracle_lib, k, n, 8, 32, 1, std=0.02)
    _compare(kt, oracle_lib, q, x, "gemm-g32", rows=tile_rows(m, rng))


TWO_ROW_SHAPES = [(896, (896, 128, 128)), (896, (4864, 4864)), (4864, (896,)), (2048, (2048, 512, 512)),
                  (2048, (8192, 8192)), (8192, (2048,)), (4096, (4096, 1024, 1024)), (4096, (14336, 14336)),
                  (14336, (4096,))]


@pytest.mark.parametrize("k,ns", TWO_ROW_SHAPES)
@pytest.mark.parametrize("bits,g", [(4, 64), (8, 32)])
def test_two_rows(kt, oracle_lib, k, ns, bits, g):
    """M = 2 (the two-row kernel) on the Qwen2-0.5B, 1B and 8B projection shapes, each
    weight alone and the weights of one input grouped. Its sums are exact in fp32 like
    the one-row kernel's, so the bound is 1e-5."""
    rng = np.random.default_rng(k + sum(ns) + bits + g)
    x = rng.standard_normal((2, k), dtype=np.float32)
    qs = [_weights(oracle_lib, k, n, bits, g, 40 + i, std=0.02) for i, n in enumerate(ns)]
    qts = [upload_quantized(kt, q) for q in qs]
    wants = [oracle_lib.multiply_quantized(x, q, 2, threads=16) for q in qs]
    for q, qt, want in zip(qs, qts, wants):
        banner("two-rows", k, q.columns, bits, g)
        got = gpu_matmul(kt, x, qt, 2)
        assert normwise_rel(got, want) <= 1e-5, normwise_rel(got, want)
    banner("two-rows grouped", k, ns, bits, g)
    outs = [kt.DeviceBuffer(2 * n * 4) for n in ns]
    kt.MatMul.multiply_quantized_group(kt.DeviceBuffer.from_numpy(x), qts, outs, 2)
    kt.synchronize()
    for o, want, n in zip(outs, wants, ns):
        got = o.download(np.float32).reshape(2, n)
        assert normwise_rel(got, want) <= 1e-5, normwise_rel(got, want)


def test_batched_rows_equal_the_row_kernel(kt, oracle_lib):
    """QuantizationTest.kt:110-134: a and W ~ U(-0.5, 0.5), INT4 g64; m copies of one row
    give that row's one-row result within 1e-4 (absolute) for every m up to 16 -- the
    reference's shape K = 300, N = 2100 (odd sizes: the generic kernels) and an aligned
    2048 x 2048 that takes the two-row kernel (m = 2) and row mode (3..16, x split into
    fp16 hi and lo parts). m >= 17 takes the prefill GEMM, whose operands are single fp16
    values: there the bound is the normwise 2e-3 criterion (the largest difference is
    printed)."""
    rng = np.random.default_rng(4)
    for k, n in ((300, 2100), (2048, 2048)):
        a = (rng.random((1, k), dtype=np.float32) - np.float32(0.5)).astype(np.float32)
        w = (rng.random((k, n), dtype=np.float32) - np.float32(0.5)).astype(np.float32)
        st, q = oracle_lib.quantize(w, 4, 64)
        assert st == 0
        qt = upload_quantized(kt, q)
        single = gpu_matmul(kt, a, qt, 1)
        assert np.abs(single - oracle_lib.multiply_quantized(a, q, 1)).max() < 1e-4
        for m in (2, 3, 5, 8, 9, 16, 17, 64):
            banner("batched", k, n, m)
            batched = gpu_matmul(kt, np.tile(a, (m, 1)), qt, m)
            diff = float(np.abs(batched - single).max())
            print(f"  max |batched - single| = {diff:.2e}", flush=True)
            if m <= 16:
                assert diff < 1e-4, (k, n, m, diff)
            else:
                assert normwise_rel(batched, np.tile(single, (m, 1))) <= TOL


LLAMA8B = [(4096, 4096), (4096, 1024), (4096, 14336), (14336, 4096)]


@pytest.mark.parametrize("bits", [4, 8])
def test_llama8b_lm_head(kt, oracle_lib, bits):
    """The Llama-3-8B head 4096 -> 128256: quantized on the device bit for bit like the
    oracle (INT4 and INT8, g64), then multiplied at M = 1, 8, 64 and 512 (rows of every
    128-row tile checked; the oracle's M = 1 row-unit kernel for one row)."""
    k, n = 4096, 128256
    rng = np.random.default_rng(50 + bits)
    banner("8b lm_head weights", bits)
    w = (rng.standard_normal((k, n), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    qt = kt.QuantizedTensor.quantize(w, k, n, kt.Quantization(bits, 64))
    st, q = oracle_lib.quantize(w, bits, 64)
    assert st == 0
    del w
    assert same_bits(qt.qdata.view(np.uint8), q.qdata), "packed bytes differ"
    assert same_bits(qt.scales, q.scales), "scales differ"
    if bits == 4:
        assert same_bits(qt.zeros.view(np.uint8), q.zeros.view(np.uint8)), "zeros differ"
    for m in (1, 8, 64, 512):
        x = rng.standard_normal((m, k), dtype=np.float32)
        banner("8b lm_head", bits, m)
        got = gpu_matmul(kt, x, qt, m)
        rows = np.arange(m) if m <= 8 else tile_rows(m, rng, every=0)
        want = oracle_lib.multiply_quantized(x[rows], q, len(rows), threads=16)
        err = normwise_rel(got[rows], want)
        print(f"  normwise={err:.3e}", flush=True)
        assert err <= (1e-5 if m <= 2 else TOL)
        if m >= 64:  # the column-run GEMM on the same rows (1002 column tiles)
            packed = gpu_matmul(kt, x, qt.pack(), m)
            qt.unpack()
            err = normwise_rel(packed[rows], want)
            print(f"  packed normwise={err:.3e}", flush=True)
            assert err <= TOL


@pytest.mark.parametrize("k,n", LLAMA8B)
@pytest.mark.parametrize("bits", [4, 8])
def test_llama8b_layers(kt, oracle_lib, k, n, bits):
    rng = np.random.default_rng(k * 3 + n + bits)
    q = _weights(oracle_lib, k, n, bits, 64, 2, std=0.02)
    qt = upload_quantized(kt, q)
    for m in (1, 8, 64, 512):
        x = rng.standard_normal((m, k), dtype=np.float32)
        banner("llama8b", k, n, bits, m)
        got = gpu_matmul(kt, x, qt, m)
        rows = np.arange(m) if m <= 8 else tile_rows(m, rng, every=64)
        want = oracle_lib.multiply_quantized(x[rows], q, len(rows), threads=16)
        err = normwise_rel(got[rows], want)
        print(f"  normwise={err:.3e}", flush=True)
        assert err <= TOL


@pytest.mark.parametrize("m", [3, 4, 8, 9, 16])
@pytest.mark.parametrize("bits,g", [(4, 64), (4, 32), (4, 128), (8, 64), (8, 32)])
def test_row_mode_small_m(kt, oracle_lib, m, bits, g):
    """3 <= M <= 16: one fp16 A row per x row, per-(row, group) powers of two; rows of
    very different magnitude (and an all-zero row) keep the 2e-3 bound; accumulate and
    alpha; strip counts that split into K-slices and the reduction kernel."""
    rng = np.random.default_rng(100 * m + 10 * bits + g)
    for k, n in [(512, 1024), (2048, 4096), (256, 272)]:
        q = _weights(oracle_lib, k, n, bits, g, 3 + m, std=0.02)
        x = rng.standard_normal((m, k)).astype(np.float32)
        x *= np.float32(10.0) ** rng.integers(-6, 6, size=(m, 1)).astype(np.float32)
        x[m // 2] = 0.0
        got, _ = _compare(kt, oracle_lib, q, x, f"rows{k}x{n}")
        again, _ = _compare(kt, oracle_lib, q, x, f"rows-again{k}x{n}")
        assert same_bits(got, again)  # K-slices meet in slice order in the reduction kernel
        c0 = rng.standard_normal((m, n)).astype(np.float32)
        _compare(kt, oracle_lib, q, x, f"rows-acc{k}x{n}", c0=c0, accumulate=True, alpha=-0.5)


def test_results_are_bit_reproducible(kt, oracle_lib):
    """Fixed-order reductions only: repeating a call gives the same bits."""
    rng = np.random.default_rng(3)
    for (k, n, bits, m) in [(4096, 14336, 4, 1), (896, 151936, 4, 1), (2048, 2048, 8, 1), (2048, 8192, 8, 512)]:
        banner("repro", k, n, bits, m)
        q = _weights(oracle_lib, k, n, bits, 64, 4, std=0.02)
        qt = upload_quantized(kt, q)
        x = rng.standard_normal((m, k), dtype=np.float32)
        first = gpu_matmul(kt, x, qt, m)
        for _ in range(2):
            assert same_bits(first, gpu_matmul(kt, x, qt, m))


def test_gemv_work_splits_agree(kt, oracle_lib):
    """Every lane width and split count of the M == 1 kernels gives the reference's result,
    and a repeat gives the same bits (every multi-slice meet adds the slices' partial sums
    in slice order, whatever order the workgroups finish in)."""
    rng = np.random.default_rng(11)
    try:
        for (k, n, bits) in [(896, 4864, 4), (4096, 1024, 8), (512, 2048, 4)]:
            q = _weights(oracle_lib, k, n, bits, 64, 5, std=0.02)
            qt = upload_quantized(kt, q)
            x = rng.standard_normal((1, k), dtype=np.float32)
            want = oracle_lib.multiply_quantized(x, q, 1)
            configs = [(1, vec, waves, splits, reduce) for vec in (4, 8) for waves in (4, 8)
                       for splits in (1, 2, 3, 5, q.groups) for reduce in (1, 2)]
            configs += [(2, 0, waves, splits, reduce) for waves in (4, 8) for splits in (1, 2, 3, 5, q.groups)
                        for reduce in (1, 2)]
            configs += [(3, 0, waves, splits, 0) for waves in (0, 2, 4, 8) for splits in (0, 1, 2, 3, 5, k // 32)]
            configs += [(4, 0, 0, 0, 0)]
            for kind, vec, waves, splits, reduce in configs:
                banner("split", k, n, bits, kind, vec, waves, splits, reduce)
                kt.MatMul.set_kernel_config(kind, vec, splits, waves, reduce)
                got = gpu_matmul(kt, x, qt, 1)
                assert normwise_rel(got, want) <= 1e-5, (kind, vec, waves, splits, reduce)
                # the in-kernel reduction leaves its counters at zero: a repeat agrees
                assert same_bits(got, gpu_matmul(kt, x, qt, 1))
    finally:
        kt.MatMul.set_kernel_config(0, 0, 0, 0, 0)


def test_quantized_linear_forward_with_bias(kt, oracle_lib):
    """QuantizedLinear.forwardInto: out = x · deq(W) + bias (QuantizedLinear.kt:22-25)."""
    rng = np.random.default_rng(12)
    for (m, k, n, bits) in [(1, 896, 4864, 4), (7, 896, 896, 8), (64, 2048, 512, 4), (3, 70, 33, 4)]:
        banner("linear", m, k, n, bits)
        w = (rng.standard_normal((k, n)) * 0.02).astype(np.float32)
        bias = rng.standard_normal(n).astype(np.float32)
        layer = kt.QuantizedLinear.from_linear(w, bias, kt.Quantization(bits, 64))
        x = rng.standard_normal((m, k)).astype(np.float32)
        out = layer.forward(kt.DeviceTensor.from_numpy(x)).numpy()
        st, q = oracle_lib.quantize(w, bits, 64)
        want = oracle_lib.multiply_quantized(x, q, m) + bias[None, :]
        assert normwise_rel(out, want) <= TOL
        # the device weight is the reference's quantization of w, bit for bit
        assert same_bits(layer.weight.qdata.view(np.uint8), q.qdata)


@pytest.mark.parametrize("m", [1, 3, 130])
def test_grouped_projections(kt, oracle_lib, m):
    """kt_qmatmul_group: q/k/v and gate/up of one input in one call, with biases."""
    rng = np.random.default_rng(17)
    for (k, ns, bits, g) in [(896, (896, 128, 128), 4, 64), (896, (4864, 4864), 4, 64), (2048, (2048, 512, 512), 8, 64),
                             (256, (64, 72, 1024, 8, 16), 4, 32)]:
        banner("group", m, k, ns, bits, g)
        qs = [_weights(oracle_lib, k, n, bits, g, 20 + i, std=0.02) for i, n in enumerate(ns)]
        qts = [upload_quantized(kt, q) for q in qs]
        x = rng.standard_normal((m, k)).astype(np.float32)
        biases = [rng.standard_normal(n).astype(np.float32) for n in ns]
        outs = [kt.DeviceBuffer.from_numpy(np.full((m, n), 3.0, np.float32)) for n in ns]
        dbias = [kt.DeviceBuffer.from_numpy(b) for b in biases]
        kt.MatMul.multiply_quantized_group(kt.DeviceBuffer.from_numpy(x), qts, outs, m, accumulate=True, alpha=0.75,
                                           biases=dbias)
        kt.synchronize()
        for q, o, b, n in zip(qs, outs, biases, ns):
            got = o.download(np.float32).reshape(m, n)
            want = oracle_lib.multiply_quantized(x, q, m, c=np.full((m, n), 3.0, np.float32), accumulate=True,
                                                 alpha=0.75) + b[None, :]
            assert normwise_rel(got, want) <= TOL
    with pytest.raises(kt.IllegalArgumentException):
        a = _weights(oracle_lib, 64, 64, 4, 64, 1)
        b = _weights(oracle_lib, 128, 64, 4, 64, 1)
        kt.MatMul.multiply_quantized_group(kt.DeviceBuffer(128 * 4), [upload_quantized(kt, a), upload_quantized(kt, b)],
                                           [kt.DeviceBuffer(256), kt.DeviceBuffer(256)], 1)


def test_unaligned_operands_take_the_generic_kernel(kt, oracle_lib):
    rng = np.random.default_rng(13)
    k, n = 256, 1024
    q = _weights(oracle_lib, k, n, 4, 64, 6, std=0.02)
    qt = upload_quantized(kt, q)
    for m in (1, 4):
        banner("unaligned", m)
        x = rng.standard_normal((m, k)).astype(np.float32)
        a = kt.DeviceBuffer(m * k * 4 + 64)
        a.upload(x, offset=4)
        c = kt.DeviceBuffer(m * n * 4 + 64)
        c.fill_zero()
        kt.MatMul.multiply_quantized(raw_ptr(a, 4), qt, raw_ptr(c, 4), m, accumulate=False)
        kt.synchronize()
        got = c.download(np.float32, m * n, offset=4).reshape(m, n)
        want = oracle_lib.multiply_quantized(x, q, m)
        assert normwise_rel(got, want) <= TOL


def test_extreme_activation_ranges(kt, oracle_lib):
    """Large and tiny activations keep full accuracy in the fp16 MFMA path."""
    rng = np.random.default_rng(14)
    k, n, m = 512, 1024, 64
    q = _weights(oracle_lib, k, n, 8, 64, 7, std=0.02)
    for scale in (1e-6, 1.0, 3e5):
        x = (rng.standard_normal((m, k)) * scale).astype(np.float32)
        _compare(kt, oracle_lib, q, x, f"xscale{scale:g}")
    tiny = _weights(oracle_lib, k, n, 4, 64, 8, std=1e-6)
    x = rng.standard_normal((m, k)).astype(np.float32)
    _compare(kt, oracle_lib, tiny, x, "tiny-weights")


def test_transposed_product(kt, oracle_lib):
    """multiplyByQuantizedTransposed (MatMul.kt:954-981)."""
    rng = np.random.default_rng(15)
    for (m, k, n, bits, g) in [(3, 130, 577, 4, 64), (5, 96, 33, 8, 64), (16, 2048, 512, 4, 32)]:
        banner("transposed", m, k, n, bits, g)
        q = _weights(oracle_lib, k, n, bits, g, 9)
        qt = upload_quantized(kt, q)
        dy = (rng.random((m, n), dtype=np.float32) - 0.5).astype(np.float32)
        dyb = kt.DeviceBuffer.from_numpy(dy)
        dx = kt.DeviceBuffer.from_numpy(np.ones((m, k), np.float32))
        kt.MatMul.multiply_by_quantized_transposed(dyb, qt, dx, m, accumulate=True)
        kt.synchronize()
        got = dx.download(np.float32).reshape(m, k)
        want = oracle_lib.multiply_by_quantized_transposed(dy, q, m, dx=np.ones((m, k), np.float32),
                                                           accumulate=True)
        assert np.abs(got - want).max() < 1e-3
        assert normwise_rel(got, want) <= TOL


def test_dequantize_rows_and_columns_exact(kt, oracle_lib):
    """dequantizeRow / dequantizeColumn / value are single fp32 products: bit-exact."""
    for (k, n, bits, g) in [(100, 37, 4, 32), (70, 9, 4, 64), (64, 130, 8, 64), (33, 40, 8, 16)]:
        banner("dequant", k, n, bits, g)
        q = _weights(oracle_lib, k, n, bits, g, 10)
        qt = upload_quantized(kt, q)
        rows = [0, k // 2, k - 1]
        got = qt.dequantize_rows(rows)
        for i, r in enumerate(rows):
            assert same_bits(got[i], q.dequantize_row(r))
        for c in (0, n // 2, n - 1):
            assert same_bits(qt.dequantize_column(c), q.dequantize_column(c))
            assert qt.value(k - 1, c) == q.value(k - 1, c)
            assert qt.raw_value(k - 1, c) == q.raw_value(k - 1, c)
        assert same_bits(qt.dequantize(), q.dequantize())


def test_linearity_at_full_size(kt, oracle_lib):
    """A size-independent property on the largest GEMV: f(x1 + x2) = f(x1) + f(x2)."""
    rng = np.random.default_rng(16)
    q = _weights(oracle_lib, 896, 151936, 4, 64, 11, std=0.02)
    qt = upload_quantized(kt, q)
    x1 = rng.standard_normal((1, 896)).astype(np.float32)
    x2 = rng.standard_normal((1, 896)).astype(np.float32)
    banner("linearity")
    y1 = gpu_matmul(kt, x1, qt, 1)
    y2 = gpu_matmul(kt, x2, qt, 1)
    y12 = gpu_matmul(kt, x1 + x2, qt, 1)
    assert normwise_rel(y12, y1.astype(np.float64) + y2) <= 1e-5
