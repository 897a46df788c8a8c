"""kt_qmatmul_noalloc: kt_qmatmul with the library's fixed device array as scratch.

Through the C ABI: two calls in a row, the second with a smaller input, give what
kt_qmatmul gives on the same operands -- bit for bit where the kernels combine their
partial sums in a fixed order (the prefill GEMM and row mode), within a normwise 1e-6
at M = 1 -- for each kernel family that uses scratch (one-row K-slice meet, row-mode
slice partials, the GEMM's prepared x); a call whose scratch would not fit the array
is refused before it launches; a recorded call replays correctly with eager work on
the same device between replays.
"""
import ctypes

import numpy as np
import pytest

from conftest import normwise_rel
from gpu_helpers import banner, same_bits, upload_quantized

pytestmark = pytest.mark.gpu


def _weights(oracle_lib, k, n, bits, g, seed):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((k, n), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    st, q = oracle_lib.quantize(w, bits, g)
    assert st == 0
    return q


def _run(kt, entry, x, qt, c0=None, accumulate=0, alpha=1.0, stream=None):
    """One call of `entry` (kt_qmatmul or kt_qmatmul_noalloc) on fresh device buffers."""
    from kotensor_amd import _lib
    m = x.shape[0]
    a = kt.DeviceBuffer.from_numpy(np.ascontiguousarray(x, dtype=np.float32))
    c = kt.DeviceBuffer(m * qt.columns * 4)
    if c0 is None:
        c.fill_zero()
    else:
        c.upload(np.ascontiguousarray(c0, dtype=np.float32))
    kt.synchronize()
    _lib.call(entry, a.ptr, m, ctypes.byref(qt.qweight), c.ptr, accumulate, ctypes.c_float(alpha), stream)
    kt.synchronize()
    return c.download(np.float32).reshape(m, qt.columns)


# (k, n, bits, g, m) of the first and the second (smaller) call, whether the kernels'
# reduction order is fixed (bit-identical results expected), and whether the weight has
# its column-run copy (2..16 rows: K-parts meeting across workgroups through the
# array's partials and counters)
CASES = [
    ("gemm", (2048, 8192, 8, 32, 512), (2048, 8192, 8, 32, 64), True, False),
    ("row mode", (4096, 14336, 4, 64, 16), (4096, 14336, 4, 64, 5), True, False),
    ("one row", (4096, 14336, 4, 64, 1), (896, 4864, 4, 64, 1), False, False),
    ("one row int8", (8192, 2048, 8, 32, 1), (2048, 2048, 8, 32, 1), False, False),
    ("packed rows", (14336, 4096, 4, 64, 16), (4096, 4096, 8, 64, 3), True, True),
]


@pytest.mark.parametrize("label,first,second,exact,packed", CASES, ids=[c[0] for c in CASES])
def test_noalloc_equals_qmatmul_on_two_calls(kt, oracle_lib, label, first, second, exact, packed):
    rng = np.random.default_rng(61)
    for k, n, bits, g, m in (first, second):
        banner("noalloc", label, k, n, bits, g, m)
        q = _weights(oracle_lib, k, n, bits, g, k + n + m)
        qt = upload_quantized(kt, q)
        if packed:
            qt = qt.pack()
        x = rng.standard_normal((m, k), dtype=np.float32)
        c0 = rng.standard_normal((m, n), dtype=np.float32)
        for acc, alpha in ((0, 1.0), (1, -0.5)):
            want = _run(kt, "kt_qmatmul", x, qt, c0, acc, alpha)
            got = _run(kt, "kt_qmatmul_noalloc", x, qt, c0, acc, alpha)
            err = normwise_rel(got, want)
            print(f"  accumulate={acc} normwise={err:.2e} same_bits={same_bits(got, want)}", flush=True)
            assert err <= 1e-6
            if exact:
                assert same_bits(got, want)
        ref = oracle_lib.multiply_quantized(x[:4], q, min(m, 4), threads=16)
        assert normwise_rel(_run(kt, "kt_qmatmul_noalloc", x, qt)[:4], ref) <= 2e-3


def test_noalloc_refuses_scratch_beyond_its_array(kt, oracle_lib):
    """The GEMM's prepared x alone (2 * M * K bytes) exceeds the 64 MiB array at
    M = 4096, K = 8192: KT_ERR_SHAPE, and the output is not touched."""
    from kotensor_amd import _lib
    q = _weights(oracle_lib, 8192, 64, 8, 32, 3)
    qt = upload_quantized(kt, q)
    m = 4096
    a = kt.DeviceBuffer(m * 8192 * 4)
    a.fill_zero()
    c = kt.DeviceBuffer.from_numpy(np.full((m, 64), 7.0, np.float32))
    kt.synchronize()
    banner("noalloc", "oversize")
    with pytest.raises(kt.IllegalArgumentException, match="fixed workspace"):
        _lib.call("kt_qmatmul_noalloc", a.ptr, m, ctypes.byref(qt.qweight), c.ptr, 0, ctypes.c_float(1.0), None)
    assert np.all(c.download(np.float32) == 7.0)


def test_noalloc_call_recorded_in_a_graph(kt, oracle_lib):
    """A recorded kt_qmatmul_noalloc (the GEMM, M = 64) replays three times with eager
    calls of both entry points on the same device between the replays; every replay
    equals the eager result."""
    from kotensor_amd import _lib
    rng = np.random.default_rng(62)
    q = _weights(oracle_lib, 2048, 2048, 4, 64, 5)
    other = _weights(oracle_lib, 2048, 512, 8, 32, 6)
    qt, ot = upload_quantized(kt, q), upload_quantized(kt, other)
    x = rng.standard_normal((64, 2048), dtype=np.float32)
    want = _run(kt, "kt_qmatmul_noalloc", x, qt)  # eager; also sets the array up
    stream = kt.Stream.create()
    a = kt.DeviceBuffer.from_numpy(x)
    c = kt.DeviceBuffer(64 * 2048 * 4)
    kt.synchronize()
    banner("noalloc", "record")
    _lib.call("kt_graph_begin", stream.handle)
    try:
        _lib.call("kt_qmatmul_noalloc", a.ptr, 64, ctypes.byref(qt.qweight), c.ptr, 0, ctypes.c_float(1.0),
                  stream.handle)
    finally:
        graph = ctypes.c_void_p()
        _lib.call("kt_graph_end", stream.handle, ctypes.byref(graph))
    try:
        for replay in range(3):
            c.fill_zero()
            kt.synchronize()
            banner("noalloc", "replay", replay)
            _lib.call("kt_graph_launch", graph, stream.handle)
            stream.synchronize()
            assert same_bits(c.download(np.float32).reshape(64, 2048), want), replay
            y = rng.standard_normal((130, 2048), dtype=np.float32)
            e1 = _run(kt, "kt_qmatmul", y, ot)
            e2 = _run(kt, "kt_qmatmul_noalloc", y, ot)
            assert same_bits(e1, e2)
    finally:
        stream.synchronize()
        _lib.call("kt_graph_destroy", graph)
        stream.destroy()
