"""The one-row product on the column-run copy (kt_qweight_pack, kt_gemv_packed.hip).

The copy is bit for bit the numpy restatement of its layout (tests/spec_numpy.py). The
product's digit sums are exact integers and its per-run combine is fp32, so it meets
the oracle's MatMul.multiplyQuantized (MatMul.kt:494-536) to a normwise 1e-5 like the
other one-row kernels (measured near 1e-7), at the Qwen2-0.5B, Llama-3.2-1B and
Llama-3-8B projection and head shapes, INT4 and INT8, g32/64/128; repeated calls give
the same bits; every split of K over waves agrees; grouped calls take biases,
accumulate and alpha; x values from 1e-30 to 1e30, zero runs and subnormals keep the
bound, and an infinite x gives non-finite outputs as the reference's sums do. Every split
of K over waves gives the same bits.
"""
import ctypes

import numpy as np
import pytest

from conftest import normwise_rel
from gpu_helpers import banner, gpu_matmul, same_bits, upload_quantized
from spec_numpy import pack_column_runs

pytestmark = pytest.mark.gpu
TOL = 1e-5


def _weights(oracle_lib, k, n, bits, g, seed, std=0.02):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((k, n), dtype=np.float32) * np.float32(std)).astype(np.float32)
    st, q = oracle_lib.quantize(w, bits, g)
    assert st == 0
    return q


def _packed(kt, q):
    return upload_quantized(kt, q).pack()


@pytest.mark.parametrize("k,n,bits,g", [(300, 2100, 4, 64), (300, 2100, 8, 32), (896, 4864, 4, 32), (128, 16, 8, 64),
                                        (200, 33, 4, 64), (4096, 1024, 8, 128), (70, 9, 4, 64), (1000, 48, 4, 96)])
def test_pack_layout_bit_exact(kt, oracle_lib, k, n, bits, g):
    q = _weights(oracle_lib, k, n, bits, g, k + n)
    banner("pack", k, n, bits, g)
    qt = _packed(kt, q)
    got = qt.packed_buffer.download(np.uint8)
    assert same_bits(got, pack_column_runs(q.qdata, k, n, bits, q.scales, q.zeros, g))


SHAPES = [(896, 896), (896, 128), (896, 4864), (4864, 896), (896, 151936), (2048, 2048), (2048, 512), (2048, 8192),
          (8192, 2048), (2048, 32000), (4096, 4096), (4096, 1024), (4096, 14336), (14336, 4096), (4096, 128256)]


@pytest.mark.parametrize("k,n", SHAPES)
@pytest.mark.parametrize("bits,g", [(4, 64), (8, 64), (4, 32), (8, 32)])
def test_packed_gemv_matches_the_oracle(kt, oracle_lib, k, n, bits, g):
    rng = np.random.default_rng(k + n + bits + g)
    q = _weights(oracle_lib, k, n, bits, g, 3)
    qt = _packed(kt, q)
    x = rng.standard_normal((1, k), dtype=np.float32)
    banner("packed", k, n, bits, g)
    got = gpu_matmul(kt, x, qt, 1)
    want = oracle_lib.multiply_quantized(x, q, 1, threads=16)
    err = normwise_rel(got, want)
    print(f"  normwise={err:.2e}", flush=True)
    assert err <= TOL
    assert same_bits(got, gpu_matmul(kt, x, qt, 1))  # repeat: same bits


def test_packed_group_sizes_and_ragged_shapes(kt, oracle_lib):
    """g from 32 to 512; K not a multiple of the 128-row chunk (the last chunk padded);
    and column counts that are not whole 16-column sets, which the other one-row
    kernels take although the weight has a packed copy."""
    rng = np.random.default_rng(5)
    for k, n, bits, g in [(512, 1008, 4, 128), (2048, 2048, 8, 128), (320, 48, 4, 32), (96, 16, 8, 32),
                          (4096, 4096, 4, 256), (1024, 4864, 8, 512), (4000, 1024, 4, 32), (512, 1000, 4, 128),
                          (320, 33, 4, 32), (96, 17, 8, 32)]:
        banner("packed-ragged", k, n, bits, g)
        q = _weights(oracle_lib, k, n, bits, g, 7)
        x = rng.standard_normal((1, k), dtype=np.float32)
        got = gpu_matmul(kt, x, _packed(kt, q), 1)
        assert normwise_rel(got, oracle_lib.multiply_quantized(x, q, 1)) <= TOL


def test_packed_work_splits_agree(kt, oracle_lib):
    """Every split of a column set's K range over 1, 2, 4 or 8 waves, with 4 or 8 KB of
    weights in flight per wave, gives the same bits (DecodeKernelTest.kt:92-109 asks the
    same of the reference's thread counts), within the bound of the oracle: K's eight
    sub-parts are summed alone and added in one fixed tree, whatever the split."""
    rng = np.random.default_rng(6)
    try:
        for k, n, bits in [(4096, 14336, 4), (896, 4864, 4), (2048, 2048, 8), (8192, 2048, 4), (16384, 1024, 8)]:
            q = _weights(oracle_lib, k, n, bits, 64, 8)
            qt = _packed(kt, q)
            x = rng.standard_normal((1, k), dtype=np.float32)
            want = oracle_lib.multiply_quantized(x, q, 1, threads=16)
            first = None
            for ring in (4, 8):
                for ks in (1, 2, 4, 8):
                    # a wave's range holds 1 to 16 chunks (other splits take another kernel)
                    if -(-k // 128) > 16 * ks or ks > -(-k // 128):
                        continue
                    banner("packed-split", k, n, bits, ring, ks)
                    kt.MatMul.set_kernel_config(5, ring, ks, 0, 0)
                    got = gpu_matmul(kt, x, qt, 1)
                    assert normwise_rel(got, want) <= TOL, (ring, ks)
                    first = got if first is None else first
                    assert same_bits(got, first), (k, n, bits, ring, ks)
    finally:
        kt.MatMul.set_kernel_config(0, 0, 0, 0, 0)


def test_packed_grouped_with_biases(kt, oracle_lib):
    rng = np.random.default_rng(9)
    for k, ns, bits, g in [(896, (896, 128, 128), 4, 64), (4096, (14336, 14336), 4, 64), (2048, (2048, 512, 512), 8, 32)]:
        banner("packed-group", k, ns, bits, g)
        qs = [_weights(oracle_lib, k, n, bits, g, 20 + i) for i, n in enumerate(ns)]
        qts = [_packed(kt, q) for q in qs]
        x = rng.standard_normal((1, k)).astype(np.float32)
        biases = [rng.standard_normal(n).astype(np.float32) for n in ns]
        outs = [kt.DeviceBuffer.from_numpy(np.full((1, n), 3.0, np.float32)) for n in ns]
        dbias = [kt.DeviceBuffer.from_numpy(b) for b in biases]
        kt.MatMul.multiply_quantized_group(kt.DeviceBuffer.from_numpy(x), qts, outs, 1, accumulate=True, alpha=0.75,
                                           biases=dbias)
        kt.synchronize()
        for q, o, b, n in zip(qs, outs, biases, ns):
            got = o.download(np.float32).reshape(1, n)
            want = oracle_lib.multiply_quantized(x, q, 1, c=np.full((1, n), 3.0, np.float32), accumulate=True,
                                                 alpha=0.75) + b[None, :]
            assert normwise_rel(got, want) <= TOL


def test_packed_activation_ranges_and_special_values(kt, oracle_lib):
    rng = np.random.default_rng(10)
    k, n = 2048, 1024
    for bits in (4, 8):
        q = _weights(oracle_lib, k, n, bits, 64, 11)
        qt = _packed(kt, q)
        cases = {}
        x = rng.standard_normal((1, k)).astype(np.float32)
        x[0, 64:96] = 0.0  # a zero run
        cases["zero-run"] = x
        for scale in (1e-30, 1e30):
            cases[f"scale{scale:g}"] = (rng.standard_normal((1, k)) * scale).astype(np.float32)
        mixed = rng.standard_normal((1, k)).astype(np.float32)
        mixed[0, ::32] *= np.float32(1e6)  # one large value per run
        cases["mixed"] = mixed
        for label, x in cases.items():
            banner("packed-range", bits, label)
            got = gpu_matmul(kt, x, qt, 1)
            want = oracle_lib.multiply_quantized(x, q, 1)
            assert np.all(np.isfinite(got)), label
            assert normwise_rel(got, want) <= TOL, (label, normwise_rel(got, want))
        # subnormal fp32 inputs: the outputs (near 1e-41) are subnormal themselves, where
        # fp32 keeps few digits; the bound is absolute, against fp64 on the dequantized weight
        sub = (rng.standard_normal((1, k)) * 1e-40).astype(np.float32)
        banner("packed-range", bits, "subnormal")
        got = gpu_matmul(kt, sub, qt, 1)
        want = sub.astype(np.float64) @ q.dequantize().astype(np.float64)
        assert np.max(np.abs(got - want)) <= 1e-43
        inf = rng.standard_normal((1, k)).astype(np.float32)
        inf[0, 100] = np.inf
        banner("packed-range", bits, "inf")
        got = gpu_matmul(kt, inf, qt, 1)
        want = oracle_lib.multiply_quantized(inf, q, 1)
        assert not np.any(np.isfinite(want))
        assert not np.any(np.isfinite(got))


def test_packed_fused_decoder_steps(kt, oracle_lib):
    """kt_rmsnorm_qmatmul_group and kt_swiglu_qmatmul on packed weights take the RMSNorm
    and the SwiGLU gate inside the product; they agree with the separate steps (the
    oracle's RMSNorm / gate, then its product) to the one-row bound."""
    from kotensor_amd import _lib
    rng = np.random.default_rng(12)
    k, h = 2048, 8192
    for bits in (4, 8):
        qs = [_weights(oracle_lib, k, n, bits, 64, 30 + i) for i, n in enumerate((2048, 512, 512))]
        qts = [_packed(kt, q) for q in qs]
        x = rng.standard_normal((1, k)).astype(np.float32)
        nw = (1 + 0.1 * rng.standard_normal(k)).astype(np.float32)
        dx, dnw = kt.DeviceBuffer.from_numpy(x), kt.DeviceBuffer.from_numpy(nw)
        normed = kt.DeviceBuffer(k * 4)
        outs = [kt.DeviceBuffer(q.columns * 4) for q in qs]
        ws = (_lib.QWeight * 3)(*[t.qweight for t in qts])
        os_ = (ctypes.c_void_p * 3)(*[o.ptr for o in outs])
        banner("packed-rmsnorm", bits)
        _lib.call("kt_rmsnorm_qmatmul_group", dx.ptr, dnw.ptr, ctypes.c_float(1e-5), normed.ptr, 1, ws, 3, os_, None, 0,
                  ctypes.c_float(1.0), None)
        kt.synchronize()
        xn = oracle_lib.rmsnorm(x, nw, 1e-5)
        for q, o in zip(qs, outs):
            want = oracle_lib.multiply_quantized(xn, q, 1)
            assert normwise_rel(o.download(np.float32).reshape(1, -1), want) <= TOL
        down = _weights(oracle_lib, h, k, bits, 64, 40)
        dt = _packed(kt, down)
        gate = rng.standard_normal((1, h)).astype(np.float32)
        up = rng.standard_normal((1, h)).astype(np.float32)
        dg, du = kt.DeviceBuffer.from_numpy(gate), kt.DeviceBuffer.from_numpy(up)
        out = kt.DeviceBuffer(k * 4)
        banner("packed-swiglu", bits)
        _lib.call("kt_swiglu_qmatmul", dg.ptr, du.ptr, 1, ctypes.byref(dt.qweight), out.ptr, 0, ctypes.c_float(1.0),
                  None, None)
        kt.synchronize()
        assert same_bits(dg.download(np.float32).reshape(1, -1), gate)  # the gate row is left as it was
        want = oracle_lib.multiply_quantized(oracle_lib.silu_mul(gate, up), down, 1)
        assert normwise_rel(out.download(np.float32).reshape(1, -1), want) <= TOL


def test_packed_swiglu_gate_pairs(kt, oracle_lib):
    """kt_rmsnorm_swiglu_gate: one launch for a row on column-run copies (each workgroup
    multiplies the same columns of gate and up and computes silu(gate) * up in its
    epilogue). Against the unfused calls (kt_rmsnorm_qmatmul_group, then kt_silu_mul): the
    same bits, since the column sums split K the same way and the gate is the same
    expression; against the oracle (RMSNorm, products, silu_mul) to the one-row bound.
    With and without RMSNorm and biases; three rows and weights without the copy take the
    unfused sequence."""
    from kotensor_amd import _lib
    rng = np.random.default_rng(40)
    for k, n, bits, g in [(2048, 8192, 4, 64), (896, 4864, 4, 64), (2048, 8192, 8, 32), (4096, 14336, 4, 64)]:
        qg, qu = _weights(oracle_lib, k, n, bits, g, 41), _weights(oracle_lib, k, n, bits, g, 42)
        tg, tu = _packed(kt, qg), _packed(kt, qu)
        nw = (1 + 0.1 * rng.standard_normal(k)).astype(np.float32)
        bg, bu = rng.standard_normal(n).astype(np.float32), rng.standard_normal(n).astype(np.float32)
        dnw, dbg, dbu = (kt.DeviceBuffer.from_numpy(v) for v in (nw, bg, bu))
        for m in (1, 3):
            x = rng.standard_normal((m, k)).astype(np.float32)
            dx = kt.DeviceBuffer.from_numpy(x)
            normed = kt.DeviceBuffer(m * k * 4)
            for use_norm, use_bias in ((True, False), (True, True), (False, False)):
                banner("swiglu-gate", k, n, bits, g, m, use_norm, use_bias)
                gate, up = kt.DeviceBuffer(m * n * 4), kt.DeviceBuffer(m * n * 4)
                _lib.call("kt_rmsnorm_swiglu_gate", dx.ptr, dnw.ptr if use_norm else None, ctypes.c_float(1e-5),
                          normed.ptr, m, ctypes.byref(tg.qweight), ctypes.byref(tu.qweight),
                          dbg.ptr if use_bias else None, dbu.ptr if use_bias else None, gate.ptr, up.ptr, None)
                # the unfused calls
                g2, u2 = kt.DeviceBuffer(m * n * 4), kt.DeviceBuffer(m * n * 4)
                ws = (_lib.QWeight * 2)(tg.qweight, tu.qweight)
                os_ = (ctypes.c_void_p * 2)(g2.ptr, u2.ptr)
                bs = (ctypes.c_void_p * 2)(dbg.ptr, dbu.ptr) if use_bias else None
                if use_norm:
                    _lib.call("kt_rmsnorm_qmatmul_group", dx.ptr, dnw.ptr, ctypes.c_float(1e-5), normed.ptr, m, ws, 2, os_,
                              bs, 0, ctypes.c_float(1.0), None)
                else:
                    _lib.call("kt_qmatmul_group", dx.ptr, m, ws, 2, os_, bs, 0, ctypes.c_float(1.0), None)
                _lib.call("kt_silu_mul", g2.ptr, u2.ptr, ctypes.c_int64(m * n), None)
                kt.synchronize()
                got_g, got_u = gate.download(np.float32).reshape(m, n), up.download(np.float32).reshape(m, n)
                assert same_bits(got_u, u2.download(np.float32).reshape(m, n))
                assert same_bits(got_g, g2.download(np.float32).reshape(m, n))
                xn = oracle_lib.rmsnorm(x, nw, 1e-5) if use_norm else x
                want_u = oracle_lib.multiply_quantized(xn, qu, m) + (bu if use_bias else 0)
                want_g = oracle_lib.multiply_quantized(xn, qg, m) + (bg if use_bias else 0)
                assert normwise_rel(got_u, want_u) <= TOL
                assert normwise_rel(got_g, oracle_lib.silu_mul(want_g.astype(np.float32), want_u.astype(np.float32))) <= 1e-4
    # a weight without the copy: the unfused sequence, same results
    k, n = 896, 4864
    qg, qu = _weights(oracle_lib, k, n, 4, 64, 43), _weights(oracle_lib, k, n, 4, 64, 44)
    x = rng.standard_normal((1, k)).astype(np.float32)
    dx = kt.DeviceBuffer.from_numpy(x)
    outs = []
    for pack in (True, False):
        tg = _packed(kt, qg) if pack else upload_quantized(kt, qg)
        tu = _packed(kt, qu)
        gate, up = kt.DeviceBuffer(n * 4), kt.DeviceBuffer(n * 4)
        _lib.call("kt_rmsnorm_swiglu_gate", dx.ptr, None, ctypes.c_float(1e-5), None, 1, ctypes.byref(tg.qweight),
                  ctypes.byref(tu.qweight), None, None, gate.ptr, up.ptr, None)
        kt.synchronize()
        outs.append(gate.download(np.float32))
    assert normwise_rel(outs[0], outs[1]) <= 1e-5
    with pytest.raises(kt.IllegalArgumentException):
        small = _packed(kt, _weights(oracle_lib, k, 128, 4, 64, 45))
        _lib.call("kt_rmsnorm_swiglu_gate", dx.ptr, None, ctypes.c_float(1e-5), None, 1, ctypes.byref(small.qweight),
                  ctypes.byref(_packed(kt, qu).qweight), None, None, kt.DeviceBuffer(n * 4).ptr,
                  kt.DeviceBuffer(n * 4).ptr, None)


# ---- 2 to 16 rows on the copy (kt_gemv_rows_packed.hip) ------------------------------

ROW_SHAPES = [(896, 896), (896, 4864), (4864, 896), (2048, 2048), (2048, 8192), (8192, 2048), (4096, 14336),
              (14336, 4096)]


@pytest.mark.parametrize("k,n", ROW_SHAPES)
@pytest.mark.parametrize("bits,g", [(4, 64), (8, 32), (4, 32), (8, 64)])
def test_packed_rows_match_the_oracle(kt, oracle_lib, k, n, bits, g):
    """2, 3, 8 and 16 rows on the copy against the oracle's tile kernel (MatMul.kt:830-881),
    row by row (rows scaled by 1e-6 .. 1e5, one row zero): x is held to 22 bits of each
    128-k chunk's largest value and the products are exact, so each row meets the oracle
    to the one-row kernels' normwise 1e-5."""
    q = _weights(oracle_lib, k, n, bits, g, 13)
    qt = _packed(kt, q)
    rng = np.random.default_rng(k + n + bits + g + 1)
    try:
        # the column-run kernel itself, also at the narrow shapes where the automatic
        # choice takes the row-block kernel
        kt.MatMul.set_kernel_config(5, 0, 0, 0, 0)
        for m in (2, 3, 8, 16):
            x = rng.standard_normal((m, k), dtype=np.float32)
            x *= (np.float32(10.0) ** rng.integers(-6, 6, size=(m, 1))).astype(np.float32)
            if m > 2:
                x[m // 2] = 0.0
            banner("packed-rows", k, n, bits, g, m)
            got = gpu_matmul(kt, x, qt, m)
            want = oracle_lib.multiply_quantized(x, q, m, threads=16)
            errs = [normwise_rel(got[r], want[r]) for r in range(m)]
            print(f"  worst row normwise={max(errs):.2e}", flush=True)
            assert max(errs) <= TOL, errs
    finally:
        kt.MatMul.set_kernel_config(0, 0, 0, 0, 0)


def test_packed_rows_do_not_depend_on_the_other_rows(kt, oracle_lib):
    """QuantizationTest.kt:110-134: a and W ~ U(-0.5, 0.5), INT4 g64; m copies of one row
    give its one-row result within 1e-4 (absolute) -- here within normwise 1e-6, since
    both sides are exact products with fp32 sums (the automatic choice, which takes small
    row counts of these weights as one-row products, and the rows kernel). Beyond the
    reference's bound, a row's bits from the rows kernel do not depend on what the other
    rows of the call hold: they are the same for every call of 2..8 rows and for every call
    of 9..16 rows (the two tile arrangements add x's hi and lo parts in different orders)."""
    rng = np.random.default_rng(41)
    try:
        for k, n in ((320, 2112), (4096, 14336)):
            a = (rng.random((1, k), dtype=np.float32) - np.float32(0.5)).astype(np.float32)
            w = (rng.random((k, n), dtype=np.float32) - np.float32(0.5)).astype(np.float32)
            st, q = oracle_lib.quantize(w, 4, 64)
            assert st == 0
            qt = _packed(kt, q)
            single = gpu_matmul(kt, a, qt, 1)
            for kind in (0, 5):
                kt.MatMul.set_kernel_config(kind, 0, 0, 0, 0)
                ref = {}
                for m in (2, 3, 5, 8, 9, 12, 16):
                    banner("packed-rows-batched", k, n, kind, m)
                    batched = gpu_matmul(kt, np.tile(a, (m, 1)), qt, m)
                    diff = float(np.abs(batched - single).max())
                    print(f"  max |batched - single| = {diff:.2e}", flush=True)
                    assert diff < 1e-4 and normwise_rel(batched, np.tile(single, (m, 1))) <= 1e-6, (k, n, m, diff)
                    if kind == 5:
                        cls = m > 8
                        ref.setdefault(cls, batched[0])
                        assert all(same_bits(batched[r], ref[cls]) for r in range(m)), m
            x = rng.standard_normal((16, k)).astype(np.float32)
            full16 = gpu_matmul(kt, x, qt, 16)
            full8 = gpu_matmul(kt, x[:8], qt, 8)
            for rows, full in (([0, 5, 7], full8), ([7, 3], full8), ([2, 6, 1, 4, 0], full8),
                               ([9, 0, 15, 3, 11, 4, 8, 13, 1, 6], full16), ([14, 2, 5, 10, 12, 7, 0, 9, 11], full16)):
                part = gpu_matmul(kt, x[rows], qt, len(rows))
                assert all(same_bits(part[i], full[r]) for i, r in enumerate(rows)), rows
    finally:
        kt.MatMul.set_kernel_config(0, 0, 0, 0, 0)


@pytest.mark.parametrize("bits,g", [(4, 64), (8, 32)])
def test_packed_rows_many_workgroups_copy_prepared_tiles(kt, oracle_lib, bits, g):
    """512 x 65536: more workgroups than CUs, where the kernel copies x tiles prepared by
    one launch instead of converting x in every workgroup. At 2, 5 and 8 rows it meets the
    oracle, and its first 4096 columns have the bits of the same columns as a weight of
    their own (few workgroups: x converted in each), whose split differs too."""
    k, n, part = 512, 65536, 4096
    rng = np.random.default_rng(47 + bits)
    w = (rng.standard_normal((k, n), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    st, q = oracle_lib.quantize(w, bits, g)
    assert st == 0
    st, qp = oracle_lib.quantize(np.ascontiguousarray(w[:, :part]), bits, g)
    assert st == 0
    del w
    qt, qtp = _packed(kt, q), _packed(kt, qp)
    try:
        kt.MatMul.set_kernel_config(5, 0, 0, 0, 0)  # the rows kernel (the 4096 columns alone are a small weight)
        for m in (2, 5, 8):
            banner("packed-rows-copy", k, n, bits, g, m)
            x = rng.standard_normal((m, k), dtype=np.float32)
            got = gpu_matmul(kt, x, qt, m)
            want = oracle_lib.multiply_quantized(x, q, m, threads=16)
            errs = [normwise_rel(got[r], want[r]) for r in range(m)]
            print(f"  worst row normwise={max(errs):.2e}", flush=True)
            assert max(errs) <= TOL, errs
            assert same_bits(gpu_matmul(kt, x, qtp, m), np.ascontiguousarray(got[:, :part])), m
    finally:
        kt.MatMul.set_kernel_config(0, 0, 0, 0, 0)


def test_packed_rows_grouped_accumulate_and_bias(kt, oracle_lib):
    """Grouped weights of one input (q/k/v, gate/up) at 2..16 rows: one preparation of x,
    a launch per weight; accumulate, alpha and biases -- on the column-run kernel (forced
    where the automatic choice takes the row-block kernel) and on the automatic choice."""
    rng = np.random.default_rng(42)
    try:
        _grouped_rows_cases(kt, oracle_lib, rng)
    finally:
        kt.MatMul.set_kernel_config(0, 0, 0, 0, 0)


def _grouped_rows_cases(kt, oracle_lib, rng):
    for m, kind in ((2, 5), (5, 5), (16, 5), (5, 0)):
        for k, ns, bits, g in [(2048, (2048, 512, 512), 8, 32), (4096, (14336, 14336), 4, 64), (896, (896, 128, 128), 4, 64)]:
            banner("packed-rows-group", m, kind, k, ns, bits, g)
            kt.MatMul.set_kernel_config(kind, 0, 0, 0, 0)
            qs = [_weights(oracle_lib, k, n, bits, g, 50 + i) for i, n in enumerate(ns)]
            qts = [_packed(kt, q) for q in qs]
            x = rng.standard_normal((m, k)).astype(np.float32)
            biases = [rng.standard_normal(n).astype(np.float32) for n in ns]
            c0 = [rng.standard_normal((m, n)).astype(np.float32) for n in ns]
            outs = [kt.DeviceBuffer.from_numpy(c) for c in c0]
            dbias = [kt.DeviceBuffer.from_numpy(b) for b in biases]
            kt.MatMul.multiply_quantized_group(kt.DeviceBuffer.from_numpy(x), qts, outs, m, accumulate=True,
                                               alpha=-0.75, biases=dbias)
            kt.synchronize()
            kt.MatMul.set_kernel_config(0, 0, 0, 0, 0)
            for q, o, b, c, n in zip(qs, outs, biases, c0, ns):
                got = o.download(np.float32).reshape(m, n)
                want = oracle_lib.multiply_quantized(x, q, m, c=c, accumulate=True, alpha=-0.75, threads=16) + b[None, :]
                assert normwise_rel(got, want) <= TOL


def test_packed_rows_work_splits_agree(kt, oracle_lib):
    """Every split of a column set's K range over 1, 2, 4 or 8 waves of one workgroup (and
    the x tiles in one phase or several) or over as many workgroups gives the same bits at
    4 and 16 rows, within the oracle's bound (inside a workgroup, a split whose x tiles do
    not fit LDS runs as the largest smaller one that does)."""
    rng = np.random.default_rng(43)
    try:
        for k, n, bits in [(4096, 14336, 4), (2048, 2048, 8), (8192, 2048, 4)]:
            q = _weights(oracle_lib, k, n, bits, 64, 44)
            qt = _packed(kt, q)
            for m in (4, 16):
                x = rng.standard_normal((m, k), dtype=np.float32)
                want = oracle_lib.multiply_quantized(x, q, m, threads=16)
                first = None
                for reduce in (1, 2):
                    for ks in (1, 2, 4, 8):
                        if -(-k // 128) > 16 * ks or ks > -(-k // 128):
                            continue
                        banner("packed-rows-split", k, n, bits, m, reduce, ks)
                        kt.MatMul.set_kernel_config(5, 0, ks, 0, reduce)
                        got = gpu_matmul(kt, x, qt, m)
                        assert normwise_rel(got, want) <= TOL, (m, reduce, ks)
                        first = got if first is None else first
                        assert same_bits(got, first), (k, n, bits, m, reduce, ks)
    finally:
        kt.MatMul.set_kernel_config(0, 0, 0, 0, 0)


# (k, n, bits, g, the most rows whose x tiles fit one workgroup holding every K-part)
@pytest.mark.parametrize("k,n,bits,g,inside_rows", [(14336, 4096, 4, 64, 8), (4096, 4096, 4, 64, 16),
                                               (4096, 1024, 8, 64, 16), (8192, 2048, 8, 32, 8),
                                               (2048, 8192, 4, 128, 16), (896, 4864, 4, 32, 16),
                                               (4096, 14336, 4, 64, 16), (14336, 4096, 4, 32, 4)])
def test_packed_rows_split_across_workgroups(kt, oracle_lib, k, n, bits, g, inside_rows):
    """The K-parts of a column set as separate workgroups that meet through memory (a
    write-through partial per wave, a counter per group of column sets, the last
    workgroup adding the parts in the tree's fixed order) against the K-parts meeting
    inside one workgroup: the same bits at every row count (one quad, two, four; hi and lo
    parts in the rows or in K), and within the oracle's bound. Two calls in a row check
    that the counters are left at zero. Where the x tiles and staged rows do not fit one
    workgroup holding every K-part (9..16 rows of K >= 8192, 5..16 rows of 14336 at g32;
    the call then goes to another kernel), the split rows are checked against the oracle
    and for not depending on the other rows of the call. 14336 -> 4096 at g32 with 9..16
    rows holds its x tiles in two phases."""
    q = _weights(oracle_lib, k, n, bits, g, 61)
    qt = _packed(kt, q)
    rng = np.random.default_rng(k + n + bits + g + 7)
    try:
        for m in (2, 3, 5, 8, 9, 12, 16):
            x = rng.standard_normal((m, k), dtype=np.float32)
            banner("packed-rows-split-wg", k, n, bits, g, m)
            kt.MatMul.set_kernel_config(5, 0, 0, 0, 2)
            across = gpu_matmul(kt, x, qt, m)
            again = gpu_matmul(kt, x, qt, m)
            assert same_bits(again, across), (k, n, bits, g, m)
            if m <= inside_rows:
                kt.MatMul.set_kernel_config(5, 0, 0, 0, 1)
                inside = gpu_matmul(kt, x, qt, m)
                assert same_bits(across, inside), (k, n, bits, g, m)
            else:  # three of the rows, with others, in a call of the same class (2..8 or 9..16)
                rows = [m - 1, 0, m // 2]
                fill = 6 if m > 8 else 2
                other = gpu_matmul(kt, np.concatenate([x[rows], x[:fill]]), qt, 3 + fill)
                assert all(same_bits(other[i], across[r]) for i, r in enumerate(rows)), (k, n, m)
            if m in (3, 5, 16):
                want = oracle_lib.multiply_quantized(x, q, m, threads=16)
                errs = [normwise_rel(across[r], want[r]) for r in range(m)]
                print(f"  worst row normwise={max(errs):.2e}", flush=True)
                assert max(errs) <= TOL, errs
    finally:
        kt.MatMul.set_kernel_config(0, 0, 0, 0, 0)


def test_packed_rows_split_grouped_accumulate_and_bias(kt, oracle_lib):
    """Grouped weights of one input across split workgroups (the counters and partials
    reused launch after launch): accumulate, alpha and biases against the oracle."""
    rng = np.random.default_rng(62)
    try:
        for m, k, ns, bits, g in [(5, 14336, (4096, 1024), 4, 64), (16, 4096, (4096, 4096, 1024), 8, 32)]:
            banner("packed-rows-split-group", m, k, ns, bits, g)
            qs = [_weights(oracle_lib, k, n, bits, g, 70 + i) for i, n in enumerate(ns)]
            qts = [_packed(kt, q) for q in qs]
            x = rng.standard_normal((m, k)).astype(np.float32)
            biases = [rng.standard_normal(n).astype(np.float32) for n in ns]
            c0 = [rng.standard_normal((m, n)).astype(np.float32) for n in ns]
            outs = [kt.DeviceBuffer.from_numpy(c) for c in c0]
            dbias = [kt.DeviceBuffer.from_numpy(b) for b in biases]
            kt.MatMul.set_kernel_config(5, 0, 0, 0, 2)
            kt.MatMul.multiply_quantized_group(kt.DeviceBuffer.from_numpy(x), qts, outs, m, accumulate=True,
                                               alpha=-0.75, biases=dbias)
            kt.synchronize()
            kt.MatMul.set_kernel_config(0, 0, 0, 0, 0)
            for q, o, b, c, n in zip(qs, outs, biases, c0, ns):
                got = o.download(np.float32).reshape(m, n)
                want = oracle_lib.multiply_quantized(x, q, m, c=c, accumulate=True, alpha=-0.75, threads=16) + b[None, :]
                assert normwise_rel(got, want) <= TOL
    finally:
        kt.MatMul.set_kernel_config(0, 0, 0, 0, 0)


@pytest.mark.parametrize("k,n,bits,g,counts", [(4096, 1024, 4, 64, (2, 5, 8, 16)), (2048, 2048, 8, 32, (2, 3, 8)),
                                               (896, 896, 4, 64, (2, 7, 16)), (8192, 2048, 4, 64, (2, 4)),
                                               (4864, 896, 4, 32, (3, 8))])
def test_packed_small_weights_rows_as_one_row_products(kt, oracle_lib, k, n, bits, g, counts):
    """Small weights at 2..16 rows run as one-row products in one launch (the automatic
    choice where the extra rows' reads cost less than the row kernels' fixed costs): each
    row's bits are its one-row result's, with accumulate and alpha, and the rows meet the
    oracle."""
    q = _weights(oracle_lib, k, n, bits, g, 81)
    qt = _packed(kt, q)
    rng = np.random.default_rng(k + n + bits + g + 9)
    for m in counts:
        banner("packed-rows-as-one-row", k, n, bits, g, m)
        x = rng.standard_normal((m, k), dtype=np.float32)
        c0 = rng.standard_normal((m, n), dtype=np.float32)
        got = gpu_matmul(kt, x, qt, m, c0, accumulate=True, alpha=-0.5)
        for r in range(m):
            one = gpu_matmul(kt, x[r:r + 1], qt, 1, c0[r:r + 1], accumulate=True, alpha=-0.5)
            assert same_bits(got[r], one[0]), (k, n, m, r)
        want = oracle_lib.multiply_quantized(x, q, m, c=c0, accumulate=True, alpha=-0.5, threads=16)
        errs = [normwise_rel(got[r], want[r]) for r in range(m)]
        print(f"  worst row normwise={max(errs):.2e}", flush=True)
        assert max(errs) <= TOL, errs


def test_packed_small_weights_grouped_rows_as_one_row_products(kt, oracle_lib):
    """Grouped small weights sharing x (q/k/v of the 1B and Qwen2 decoders) at 2..8 rows,
    as one-row products in one launch: each row's bits are its one-row grouped result's,
    with accumulate, alpha and biases, and they meet the oracle."""
    rng = np.random.default_rng(83)
    for k, ns, bits, g, counts in [(2048, (2048, 512, 512), 4, 64, (2, 4)), (896, (896, 128, 128), 4, 64, (3, 8)),
                                   (2048, (2048, 512, 512), 8, 32, (2, 3))]:
        qs = [_weights(oracle_lib, k, n, bits, g, 90 + i) for i, n in enumerate(ns)]
        qts = [_packed(kt, q) for q in qs]
        biases = [rng.standard_normal(n).astype(np.float32) for n in ns]
        dbias = [kt.DeviceBuffer.from_numpy(b) for b in biases]
        for m in counts:
            banner("packed-group-rows-as-one-row", k, ns, bits, g, m)
            x = rng.standard_normal((m, k)).astype(np.float32)
            c0 = [rng.standard_normal((m, n)).astype(np.float32) for n in ns]

            def run(xs, cs, rows):
                outs = [kt.DeviceBuffer.from_numpy(np.ascontiguousarray(c)) for c in cs]
                kt.MatMul.multiply_quantized_group(kt.DeviceBuffer.from_numpy(np.ascontiguousarray(xs)), qts, outs,
                                                   rows, accumulate=True, alpha=-0.75, biases=dbias)
                kt.synchronize()
                return [o.download(np.float32).reshape(rows, n) for o, n in zip(outs, ns)]

            got = run(x, c0, m)
            for r in range(m):
                one = run(x[r:r + 1], [c[r:r + 1] for c in c0], 1)
                assert all(same_bits(gw[r], ow[0]) for gw, ow in zip(got, one)), (k, ns, m, r)
            for q, o, b, c in zip(qs, got, biases, c0):
                want = oracle_lib.multiply_quantized(x, q, m, c=c, accumulate=True, alpha=-0.75, threads=16) + b[None, :]
                assert normwise_rel(o, want) <= TOL
