"""kt_qmatmul_chain: dependent one-row products as one launch (gemv_chain_kernel).

The steps of a decoder layer between two attention calls (TransformerBlock.kt:40-46:
wOut with its residual add, norm2 with the SwiGLU gate pair, the down projection with
its residual add, the next layer's norm1 with q/k/v, or the final norm and the head),
each reading what earlier steps wrote and writing what earlier steps read. A chained
stage runs the same kernel body as the step's own call (only the order of its loads and
the device counters between stages differ), so every output equals the separate calls'
bit for bit; the counters return to zero, so launches in a row keep giving those bits.
Weights without the column-run copy take the separate calls.
"""
import ctypes

import numpy as np
import pytest

from gpu_helpers import banner, same_bits, upload_quantized

pytestmark = pytest.mark.gpu


def _weight(kt, oracle_lib, k, n, bits, g, seed, pack=True):
    rng = np.random.default_rng(seed)
    st, q = oracle_lib.quantize((rng.standard_normal((k, n)) * 0.02).astype(np.float32), bits, g)
    assert st == 0
    t = upload_quantized(kt, q)
    return t.pack() if pack else t


class Layer:
    """Device buffers and weights of one decoder layer's projections (one token)."""

    def __init__(self, kt, oracle_lib, dim, hidden, kv, bits, g, seed, qkv_bias=False, head=0, pack=True):
        rng = np.random.default_rng(seed)
        self.kt, self.dim, self.hidden, self.kv, self.head = kt, dim, hidden, kv, head
        W = lambda k, n, s: _weight(kt, oracle_lib, k, n, bits, g, seed * 16 + s, pack)
        self.wo, self.wg, self.wu, self.wd = W(dim, dim, 1), W(dim, hidden, 2), W(dim, hidden, 3), W(hidden, dim, 4)
        self.wq, self.wk, self.wv = W(dim, dim, 5), W(dim, kv, 6), W(dim, kv, 7)
        self.wh = W(dim, head, 8) if head else None
        self.norm2 = (1 + 0.1 * rng.standard_normal(dim)).astype(np.float32)
        self.norm1 = (1 + 0.1 * rng.standard_normal(dim)).astype(np.float32)
        self.biases = [rng.standard_normal(n).astype(np.float32) for n in (dim, kv, kv)] if qkv_bias else None
        self.init = {"x": rng.standard_normal(dim).astype(np.float32),
                     "ctx": rng.standard_normal(dim).astype(np.float32)}
        self.dev = {}

    def reset(self):
        """Fresh device state: x and the attention context as drawn, every output zeroed."""
        kt = self.kt
        d = self.dev
        d["x"] = kt.DeviceBuffer.from_numpy(self.init["x"])
        d["ctx"] = kt.DeviceBuffer.from_numpy(self.init["ctx"])
        for name, n in (("gate", self.hidden), ("up", self.hidden), ("q", self.dim), ("k", self.kv), ("v", self.kv),
                        ("logits", self.head), ("normed", self.dim)):
            if n:
                d[name] = kt.DeviceBuffer.from_numpy(np.zeros(n, np.float32))
        d["norm1"] = kt.DeviceBuffer.from_numpy(self.norm1)
        d["norm2"] = kt.DeviceBuffer.from_numpy(self.norm2)
        if self.biases:
            d["b"] = [kt.DeviceBuffer.from_numpy(b) for b in self.biases]

    def steps(self):
        """(x, norm, weights, outputs, biases, accumulate, swiglu) of each step."""
        d = self.dev
        qkv_b = [b.ptr for b in d["b"]] if self.biases else None
        out = [(d["ctx"], None, [self.wo], [d["x"]], None, 1, 0),
               (d["x"], d["norm2"], [self.wg, self.wu], [d["gate"], d["up"]], None, 0, 1),
               (d["gate"], None, [self.wd], [d["x"]], None, 1, 0),
               (d["x"], d["norm1"], [self.wq, self.wk, self.wv], [d["q"], d["k"], d["v"]], qkv_b, 0, 0)]
        if self.head:
            out.append((d["x"], d["norm1"], [self.wh], [d["logits"]], None, 0, 0))
        return out

    def results(self):
        self.kt.synchronize()
        return {k: v.download(np.float32) for k, v in self.dev.items()
                if k in ("x", "gate", "up", "q", "k", "v", "logits")}


def _struct(kt, layer):
    from kotensor_amd import _lib
    keep = []
    steps = (_lib.QMatmulStep * len(layer.steps()))()
    for i, (x, nw, ws, outs, biases, acc, swiglu) in enumerate(layer.steps()):
        wa = (_lib.QWeight * len(ws))(*[w.qweight for w in ws])
        oa = (ctypes.c_void_p * len(outs))(*[o.ptr for o in outs])
        ba = (ctypes.c_void_p * len(ws))(*biases) if biases else None
        keep += [wa, oa, ba]
        s = steps[i]
        s.x, s.norm_weight, s.eps = x.ptr, nw.ptr if nw is not None else None, 1e-5
        s.normed = layer.dev["normed"].ptr
        s.weights = ctypes.cast(wa, ctypes.POINTER(_lib.QWeight))
        s.count = len(ws)
        s.outputs = ctypes.cast(oa, ctypes.POINTER(ctypes.c_void_p))
        s.biases = ctypes.cast(ba, ctypes.POINTER(ctypes.c_void_p)) if ba is not None else None
        s.accumulate, s.alpha, s.swiglu_gate = acc, 1.0, swiglu
    return steps, keep


def _separate(kt, layer):
    """The same steps as their own calls."""
    from kotensor_amd import _lib
    for x, nw, ws, outs, biases, acc, swiglu in layer.steps():
        if swiglu:
            _lib.call("kt_rmsnorm_swiglu_gate", x.ptr, nw.ptr, ctypes.c_float(1e-5), layer.dev["normed"].ptr, 1,
                      ctypes.byref(ws[0].qweight), ctypes.byref(ws[1].qweight), None, None, outs[0].ptr, outs[1].ptr,
                      None)
            continue
        wa = (_lib.QWeight * len(ws))(*[w.qweight for w in ws])
        oa = (ctypes.c_void_p * len(outs))(*[o.ptr for o in outs])
        ba = (ctypes.c_void_p * len(ws))(*biases) if biases else None
        if nw is not None:
            _lib.call("kt_rmsnorm_qmatmul_group", x.ptr, nw.ptr, ctypes.c_float(1e-5), layer.dev["normed"].ptr, 1, wa,
                      len(ws), oa, ba, acc, ctypes.c_float(1.0), None)
        else:
            _lib.call("kt_qmatmul_group", x.ptr, 1, wa, len(ws), oa, ba, acc, ctypes.c_float(1.0), None)


def _chained(kt, layer):
    from kotensor_amd import _lib
    steps, keep = _struct(kt, layer)
    _lib.call("kt_qmatmul_chain", steps, len(steps), None)
    return keep


CASES = [  # dim, hidden, kv, bits, g, qkv bias, head
    (2048, 8192, 512, 4, 64, False, 0),  # Llama-3.2-1B
    (2048, 8192, 512, 8, 32, False, 0),
    (896, 4864, 128, 4, 64, True, 151936),  # Qwen2-0.5B, the last layer with the head
    (896, 4864, 128, 4, 32, True, 151936),  # the same at the group size of 32
    (896, 4864, 128, 8, 32, True, 151936),
    (4096, 14336, 1024, 4, 64, False, 0),  # Llama-3-8B
]


@pytest.mark.parametrize("dim,hidden,kv,bits,g,bias,head", CASES)
def test_chain_equals_the_separate_calls(kt, oracle_lib, dim, hidden, kv, bits, g, bias, head):
    layer = Layer(kt, oracle_lib, dim, hidden, kv, bits, g, 7, qkv_bias=bias, head=head)
    banner("chain", dim, hidden, kv, bits, g, bias, head)
    layer.reset()
    _separate(kt, layer)
    want = layer.results()
    for rep in range(3):
        layer.reset()
        keep = _chained(kt, layer)
        got = layer.results()
        del keep
        for k in want:
            assert same_bits(got[k], want[k]), (rep, k)


def test_chain_launches_in_a_row(kt, oracle_lib):
    """Fifty chains back to back on one stream, each checked: the counters a chain leaves
    are the zeros the next one needs."""
    layer = Layer(kt, oracle_lib, 2048, 8192, 512, 4, 64, 8)
    layer.reset()
    _separate(kt, layer)
    want = layer.results()
    from kotensor_amd import _lib
    banner("chain x50")
    for rep in range(50):
        layer.reset()
        steps, keep = _struct(kt, layer)
        _lib.call("kt_qmatmul_chain", steps, len(steps), None)
        got = layer.results()
        assert all(same_bits(got[k], want[k]) for k in want), rep


def test_chain_without_the_copy_and_argument_checks(kt, oracle_lib):
    from kotensor_amd import _lib
    layer = Layer(kt, oracle_lib, 896, 4864, 128, 4, 64, 9, pack=False)
    banner("chain unpacked")
    layer.reset()
    _separate(kt, layer)
    want = layer.results()
    layer.reset()
    keep = _chained(kt, layer)
    got = layer.results()
    del keep
    assert all(same_bits(got[k], want[k]) for k in want)
    steps, keep = _struct(kt, layer)
    with pytest.raises(kt.IllegalArgumentException):
        _lib.call("kt_qmatmul_chain", steps, 0, None)
    with pytest.raises(kt.IllegalArgumentException):
        _lib.call("kt_qmatmul_chain", steps, 7, None)
    steps[1].count = 3  # the SwiGLU pair takes two weights
    with pytest.raises(kt.IllegalArgumentException):
        _lib.call("kt_qmatmul_chain", steps, 4, None)


def test_a_wait_that_gives_up_is_reported(kt, oracle_lib):
    """A chained stage whose input never arrives (the test hook makes every stage withhold
    its partition flags) gives up after a small poll budget; every kernel still exits,
    the stream's next synchronization raises IllegalStateException once, and the
    stream's counters are clear again: the next chain gives the separate calls' bits."""
    from kotensor_amd import _lib
    layer = Layer(kt, oracle_lib, 896, 4864, 128, 4, 64, 10)
    layer.reset()
    _separate(kt, layer)
    want = layer.results()
    banner("chain give-up")
    layer.reset()
    steps, keep = _struct(kt, layer)
    _lib.call("kt_debug_wait_limits", 64, 1)
    try:
        _lib.call("kt_qmatmul_chain", steps, len(steps), None)
    finally:
        _lib.call("kt_debug_wait_limits", 0, 0)
    with pytest.raises(kt.IllegalStateException, match="gave up"):
        kt.synchronize()
    kt.synchronize()  # reported once
    with pytest.raises(kt.IllegalArgumentException):
        _lib.call("kt_debug_wait_limits", 0, 2)
    layer.reset()
    steps, keep = _struct(kt, layer)
    _lib.call("kt_qmatmul_chain", steps, len(steps), None)
    got = layer.results()
    del keep
    assert all(same_bits(got[k], want[k]) for k in want)
