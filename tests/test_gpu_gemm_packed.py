"""The prefill GEMM on the column-run copy (gemm_packed_kernel in kt_gemm.hip).

A weight with its column-run copy (kt_qweight_pack) and a group size that is a multiple of
32 takes this kernel for M >= 17 (smaller M go to the one-row and few-row kernels;
MatMul.multiplyQuantized's M > 1 branch,
MatMul.kt:479-485 -> computeQuantizedTile :830-881). Its operands are the fp16 values the
other prefill GEMM uses (a scaled per row by a power of two, (q - zero) * scale rounded
once), so it meets the oracle to the same normwise 2e-3 (measured near 3e-4), on every
row tile; K is split across workgroups when the tiles alone do not fill the GPU; ragged
M, N and K, biases, accumulate and alpha, grouped weights, extreme activation ranges,
and repeated calls giving the same bits.
"""
import numpy as np
import pytest

from conftest import normwise_rel
from gpu_helpers import banner, gpu_matmul, same_bits, upload_quantized

pytestmark = pytest.mark.gpu
TOL = 2e-3


def _weights(oracle_lib, k, n, bits, g, seed, std=0.02):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((k, n), dtype=np.float32) * np.float32(std)).astype(np.float32)
    st, q = oracle_lib.quantize(w, bits, g)
    assert st == 0
    return q


def _rows(m, rng):
    """Every row up to 512; otherwise the first, last and a random row of every 128-row tile."""
    if m <= 512:
        return np.arange(m)
    tiles = np.arange(0, m, 128)
    picks = [tiles, np.minimum(tiles + 127, m - 1), np.minimum(tiles + rng.integers(1, 127, tiles.size), m - 1)]
    return np.unique(np.concatenate(picks))


def _check(kt, oracle_lib, q, x, label, c0=None, accumulate=False, alpha=1.0):
    m = x.shape[0]
    rng = np.random.default_rng(m)
    banner("gemm-packed", label, f"M={m}", f"K={q.rows}", f"N={q.columns}", f"int{q.bits}/g{q.group_size}")
    qt = upload_quantized(kt, q).pack()
    got = gpu_matmul(kt, x, qt, m, c0=c0, accumulate=accumulate, alpha=alpha)
    idx = _rows(m, rng)
    want = oracle_lib.multiply_quantized(x[idx], q, len(idx), c=None if c0 is None else c0[idx], accumulate=accumulate,
                                         alpha=alpha, threads=16)
    err = normwise_rel(got[idx], want)
    print(f"  normwise={err:.3e}", flush=True)
    assert err <= TOL, (label, err)
    return qt, got


LLAMA1B = [(2048, 2048), (2048, 512), (2048, 8192), (8192, 2048)]


@pytest.mark.parametrize("k,n", LLAMA1B)
@pytest.mark.parametrize("m", [17, 64, 128, 512])
@pytest.mark.parametrize("bits,g", [(8, 32), (4, 32), (8, 128), (4, 64)])
def test_packed_gemm_matches_the_oracle(kt, oracle_lib, m, k, n, bits, g):
    rng = np.random.default_rng(m + k + n + bits + g)
    x = rng.standard_normal((m, k), dtype=np.float32)
    q = _weights(oracle_lib, k, n, bits, g, 3)
    qt, got = _check(kt, oracle_lib, q, x, "llama1b")
    assert same_bits(got, gpu_matmul(kt, x, qt, m))  # repeat: same bits


LLAMA8B = [(4096, 4096), (4096, 1024), (4096, 14336), (14336, 4096)]


@pytest.mark.parametrize("k,n", LLAMA8B)
@pytest.mark.parametrize("m", [64, 512])
@pytest.mark.parametrize("bits", [4, 8])
def test_packed_gemm_llama8b_shapes(kt, oracle_lib, m, k, n, bits):
    """The Llama-3-8B projection shapes at the prefill row counts the bench times (g64,
    the reference's default group), every row of every tile against the oracle."""
    rng = np.random.default_rng(m + k + n + bits)
    x = rng.standard_normal((m, k), dtype=np.float32)
    q = _weights(oracle_lib, k, n, bits, 64, 11)
    _check(kt, oracle_lib, q, x, "llama8b")


def test_packed_gemm_large_shapes(kt, oracle_lib):
    """The Llama-3-8B FFN and the Qwen2 shapes at prefill sizes, rows of every tile."""
    rng = np.random.default_rng(21)
    for m, k, n, bits, g in [(2048, 4096, 14336, 8, 32), (1024, 14336, 4096, 4, 64), (640, 896, 4864, 4, 32),
                             (256, 4864, 896, 8, 64)]:
        x = rng.standard_normal((m, k), dtype=np.float32)
        _check(kt, oracle_lib, _weights(oracle_lib, k, n, bits, g, 4), x, "large")


def test_packed_gemm_ragged_shapes(kt, oracle_lib):
    """M, N and K that are not whole tiles (the copy's padding is zero and its trailing
    columns are dropped), group sizes up to 512, a last group shorter than g."""
    rng = np.random.default_rng(22)
    for m, k, n, bits, g in [(5, 130, 584, 8, 32), (131, 200, 136, 4, 32), (300, 1000, 1000, 8, 64),
                             (129, 4000, 1032, 4, 32), (70, 512, 4864, 8, 512), (3, 96, 8, 4, 32),
                             (260, 2112, 2056, 8, 96)]:
        x = rng.standard_normal((m, k), dtype=np.float32)
        _check(kt, oracle_lib, _weights(oracle_lib, k, n, bits, g, 5), x, "ragged")


def test_packed_gemm_accumulate_alpha_and_split_k(kt, oracle_lib):
    """accumulate and alpha on the direct path and on the split-K path (a small tile grid
    splits K across workgroups and gemm_reduce adds the slices in order)."""
    rng = np.random.default_rng(23)
    for m, k, n in [(512, 2048, 8192), (3, 2048, 512), (64, 8192, 256)]:
        x = rng.standard_normal((m, k), dtype=np.float32)
        c0 = rng.standard_normal((m, n), dtype=np.float32)
        q = _weights(oracle_lib, k, n, 8, 32, 6)
        _check(kt, oracle_lib, q, x, "acc", c0=c0, accumulate=True, alpha=0.75)


def test_packed_gemm_grouped_with_biases(kt, oracle_lib):
    rng = np.random.default_rng(24)
    for m in (3, 130):
        for k, ns, bits, g in [(896, (896, 128, 128), 4, 64), (2048, (2048, 512, 512), 8, 32), (2048, (8192, 8192), 4, 32)]:
            banner("gemm-packed-group", m, k, ns, bits, g)
            qs = [_weights(oracle_lib, k, n, bits, g, 30 + i) for i, n in enumerate(ns)]
            qts = [upload_quantized(kt, q).pack() for q in qs]
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
                                                     alpha=0.75, threads=16) + b[None, :]
                assert normwise_rel(got, want) <= TOL


def test_packed_gemm_extreme_ranges(kt, oracle_lib):
    """Large and tiny activations, tiny weight scales: the per-row and per-weight powers
    of two keep the fp16 operands in range."""
    rng = np.random.default_rng(25)
    k, n, m = 512, 1024, 64
    q = _weights(oracle_lib, k, n, 8, 64, 7)
    for scale in (1e-6, 1.0, 3e5):
        x = (rng.standard_normal((m, k)) * scale).astype(np.float32)
        _check(kt, oracle_lib, q, x, f"xscale{scale:g}")
    x = rng.standard_normal((m, k)).astype(np.float32)
    _check(kt, oracle_lib, _weights(oracle_lib, k, n, 4, 64, 8, std=1e-6), x, "tiny-weights")
    zero_rows = rng.standard_normal((m, k)).astype(np.float32)
    zero_rows[5] = 0.0
    _check(kt, oracle_lib, q, zero_rows, "zero-row")


def test_packed_and_plain_gemm_agree(kt, oracle_lib):
    """The same weight with and without its copy: the two GEMMs take the same fp16
    operands and differ only in the order of the fp32 sums."""
    rng = np.random.default_rng(26)
    for bits, g in ((8, 32), (4, 64)):
        k, n, m = 2048, 2048, 256
        q = _weights(oracle_lib, k, n, bits, g, 9)
        x = rng.standard_normal((m, k)).astype(np.float32)
        banner("gemm-packed-vs-plain", bits, g)
        plain = gpu_matmul(kt, x, upload_quantized(kt, q), m)
        packed = gpu_matmul(kt, x, upload_quantized(kt, q).pack(), m)
        assert normwise_rel(packed, plain) <= 1e-5


def test_int8_with_zero_points(kt, oracle_lib):
    """INT8 weights carrying zero points (the quantizer writes none for INT8, but a
    QuantizedTensor may hold them: value = (q - zero) * scale with q and zero signed):
    gemm_packed_kernel<8, true> and the reference-layout GEMM against the oracle, and the
    one-row kernel on the copy, at g32 and g64 with ragged N."""
    from oracle import Quantized
    rng = np.random.default_rng(27)
    for m, k, n, g in [(512, 2048, 1024, 32), (130, 1000, 584, 64), (1, 2048, 2048, 64)]:
        groups = -(-k // g)
        qdata = rng.integers(-128, 128, size=k * n, dtype=np.int64).astype(np.int8)
        scales = (rng.random(groups * n, dtype=np.float32) * 0.02 + 0.001).astype(np.float32)
        zeros = rng.integers(-20, 21, size=groups * n, dtype=np.int64).astype(np.int8)
        q = Quantized(qdata, scales, zeros, k, n, 8, g)
        x = rng.standard_normal((m, k), dtype=np.float32)
        want = oracle_lib.multiply_quantized(x, q, m, threads=16)
        banner("int8-zp", m, k, n, g)
        plain = gpu_matmul(kt, x, upload_quantized(kt, q), m)
        packed = gpu_matmul(kt, x, upload_quantized(kt, q).pack(), m)
        tol = 1e-5 if m == 1 else TOL  # the one-row kernel sums exactly; the GEMMs round to fp16
        assert normwise_rel(packed, want) <= tol, normwise_rel(packed, want)
        assert normwise_rel(plain, want) <= tol, normwise_rel(plain, want)
