"""The oracle: a CPU restatement of Kotensor's group-wise INT8/INT4 quantization
path (kt_oracle.c), with a numpy interface.

TEST INFRASTRUCTURE ONLY. Only tests/, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of bench.py use it, as the checker and the CPU baseline. The
product (kotensor_amd / libkotensor_hip.so) never imports or links it.

Pinning status of each function is listed in kt_oracle.h.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIBRARY_PATH = HERE / "_build" / "libkt_oracle.so"
# The same source built with FMA contraction and AVX2: a CPU baseline, never a checker.
FAST_LIBRARY_PATH = HERE / "_build" / "libkt_oracle_fast.so"

KO_OK = 0
KO_ERR_ARG = -1
KO_ERR_NAN = -3


class QW(ctypes.Structure):
    _fields_ = [
        ("qdata", ctypes.c_void_p),
        ("scales", ctypes.c_void_p),
        ("zeros", ctypes.c_void_p),
        ("rows", ctypes.c_int32),
        ("columns", ctypes.c_int32),
        ("bits", ctypes.c_int32),
        ("group_size", ctypes.c_int32),
    ]


_lib = None


def build() -> Path:
    """Compiles the oracle with its Makefile (gcc, -ffp-contract=off)."""
    proc = subprocess.run(["make", "-s", "-C", str(HERE)], capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{proc.stdout}\n{proc.stderr}")
    return LIBRARY_PATH


def lib():
    global _lib
    if _lib is None:
        if not LIBRARY_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIBRARY_PATH))
        P, I, F = ctypes.c_void_p, ctypes.c_int32, ctypes.c_float
        L.ko_groups.argtypes = [I, I]
        L.ko_bytes_per_row.argtypes = [I, I]
        L.ko_java_round.argtypes = [F, ctypes.POINTER(I)]
        L.ko_quantize.argtypes = [P, I, I, I, I, P, P, P]
        L.ko_raw_value.argtypes = [ctypes.POINTER(QW), I, I]
        L.ko_value.argtypes = [ctypes.POINTER(QW), I, I]
        L.ko_value.restype = F
        L.ko_dequantize_row.argtypes = [ctypes.POINTER(QW), I, P]
        L.ko_dequantize_row.restype = None
        L.ko_dequantize_column.argtypes = [ctypes.POINTER(QW), I, P]
        L.ko_dequantize_column.restype = None
        L.ko_multiply_quantized.argtypes = [P, ctypes.POINTER(QW), P, I, I, F, I]
        L.ko_multiply_by_quantized_transposed.argtypes = [P, ctypes.POINTER(QW), P, I, I, I]
        L.ko_row_units.argtypes = [ctypes.POINTER(QW), P]
        L.ko_row_units.restype = None
        L.ko_rope_inv_freq.argtypes = [I, F, F, F, F, I, P]
        L.ko_rope_inv_freq.restype = None
        L.ko_rmsnorm.argtypes = [P, I, I, P, F, P]
        L.ko_rmsnorm.restype = None
        L.ko_rope_rows.argtypes = [P, I, I, I, P, I]
        L.ko_rope_rows.restype = None
        L.ko_attend.argtypes = [P, I, I, P, P, I, I, I, I, I, P, P]
        L.ko_attend.restype = None
        L.ko_silu_mul.argtypes = [P, P, I]
        L.ko_silu_mul.restype = None
        L.ko_argmax.argtypes = [P, I]
        L.ko_fused_cross_entropy.argtypes = [P, I, ctypes.POINTER(QW), P, P, I, P, P, P, I]
        _lib = L
    return _lib


_fast = None


def fast_lib():
    """The contracted (FMA, AVX2) build, for the CPU baseline's "fast" figure only."""
    global _fast
    if _fast is None:
        if not FAST_LIBRARY_PATH.exists():
            build()
        L = ctypes.CDLL(str(FAST_LIBRARY_PATH))
        L.ko_multiply_quantized.argtypes = [ctypes.c_void_p, ctypes.POINTER(QW), ctypes.c_void_p, ctypes.c_int32,
                                            ctypes.c_int32, ctypes.c_float, ctypes.c_int32]
        _fast = L
    return _fast


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def groups(rows: int, group_size: int) -> int:
    return lib().ko_groups(rows, group_size)


def bytes_per_row(columns: int, bits: int) -> int:
    return lib().ko_bytes_per_row(columns, bits)


def java_round(x: float) -> tuple[int, bool]:
    nan = ctypes.c_int32(0)
    r = lib().ko_java_round(ctypes.c_float(x), ctypes.byref(nan))
    return int(r), bool(nan.value)


class Quantized:
    """Host arrays of one quantized tensor in the reference layout."""

    def __init__(self, qdata, scales, zeros, rows, columns, bits, group_size):
        self.qdata = np.ascontiguousarray(qdata).view(np.uint8).reshape(-1)
        self.scales = np.ascontiguousarray(scales, dtype=np.float32).reshape(-1)
        self.zeros = None if zeros is None else np.ascontiguousarray(zeros).view(np.int8).reshape(-1)
        self.rows, self.columns, self.bits, self.group_size = int(rows), int(columns), int(bits), int(group_size)
        self.groups = groups(self.rows, self.group_size)
        self.bytes_per_row = bytes_per_row(self.columns, self.bits)
        self._qw = QW(_p(self.qdata).value, _p(self.scales).value,
                      None if self.zeros is None else _p(self.zeros).value,
                      self.rows, self.columns, self.bits, self.group_size)

    @property
    def qw(self) -> QW:
        return self._qw

    def raw_value(self, row, column) -> int:
        return int(lib().ko_raw_value(ctypes.byref(self._qw), row, column))

    def value(self, row, column) -> float:
        return float(lib().ko_value(ctypes.byref(self._qw), row, column))

    def dequantize_row(self, row) -> np.ndarray:
        out = np.empty(self.columns, dtype=np.float32)
        lib().ko_dequantize_row(ctypes.byref(self._qw), row, _p(out))
        return out

    def dequantize_column(self, column) -> np.ndarray:
        out = np.empty(self.rows, dtype=np.float32)
        lib().ko_dequantize_column(ctypes.byref(self._qw), column, _p(out))
        return out

    def dequantize(self) -> np.ndarray:
        """value(r, c) for every element as fp32 [rows x columns] (QuantizedTensor.kt:172-186,
        243-249): scale * (raw - zero), the integer difference taken before the one fp32
        product, as dequantize_row does in C. Vectorised with numpy; equal to
        dequantize_row row for row (tests/test_oracle_quantize.py checks it bit for bit)."""
        k, n, bpr = self.rows, self.columns, self.bytes_per_row
        q = self.qdata.reshape(k, bpr)
        if self.bits == 8:
            raw = q.view(np.int8).astype(np.int32)
        else:
            raw = np.empty((k, n), dtype=np.int32)
            raw[:, :bpr] = q[:, :bpr] & 0xF
            raw[:, bpr:] = (q[:, :n - bpr] >> 4) & 0xF
        gidx = np.arange(k) // self.group_size
        if self.zeros is not None:
            raw -= self.zeros.reshape(self.groups, n)[gidx].astype(np.int32)
        return (self.scales.reshape(self.groups, n)[gidx] * raw.astype(np.float32)).astype(np.float32)

    def row_units(self) -> list[int]:
        out = np.zeros(6, dtype=np.int32)
        lib().ko_row_units(ctypes.byref(self._qw), _p(out))
        return [int(v) for v in out]


def quantize(data: np.ndarray, bits: int, group_size: int) -> tuple[int, Quantized]:
    """(status, Quantized) for fp32 ``data`` ``[rows x columns]`` (QuantizedTensor.kt:261-324)."""
    data = np.ascontiguousarray(data, dtype=np.float32)
    rows, columns = data.shape
    g = groups(rows, group_size)
    bpr = bytes_per_row(columns, bits)
    q = np.empty(rows * bpr, dtype=np.uint8)
    s = np.empty(g * columns, dtype=np.float32)
    z = np.empty(g * columns, dtype=np.int8) if bits == 4 else None
    status = lib().ko_quantize(_p(data), rows, columns, bits, group_size, _p(q), _p(s), _p(z))
    return int(status), Quantized(q, s, z, rows, columns, bits, group_size)


def multiply_quantized(a: np.ndarray, w: Quantized, m: int, c: np.ndarray | None = None, accumulate: bool = False,
                       alpha: float = 1.0, threads: int = 1, fast: bool = False) -> np.ndarray:
    """MatMul.multiplyQuantized (MatMul.kt:460-486), returning c ``[m x N]``; fast=True
    runs the contracted build (CPU baseline timing only: its sums round differently)."""
    a = np.ascontiguousarray(a, dtype=np.float32).reshape(-1)
    if c is None:
        c = np.zeros(m * w.columns, dtype=np.float32)
    c = np.ascontiguousarray(c, dtype=np.float32).reshape(-1).copy()
    st = (fast_lib() if fast else lib()).ko_multiply_quantized(_p(a), ctypes.byref(w.qw), _p(c), m, int(accumulate),
                                                               ctypes.c_float(alpha), threads)
    if st != KO_OK:
        raise ValueError(f"oracle multiply_quantized status {st}")
    return c.reshape(m, w.columns)


def fused_cross_entropy(hidden: np.ndarray, w: Quantized, targets, bias: np.ndarray | None = None,
                        ignore_index: int = -100, grads: bool = True, threads: int = 1):
    """fusedCrossEntropyLoss with a quantized head (Loss.kt:114-219): returns (loss,
    hidden_grad [rows x K], bias_grad [N]) for an upstream gradient of 1, the gradients
    None when grads is False. Raises ValueError where the reference's require fails."""
    hidden = np.ascontiguousarray(hidden, dtype=np.float32).reshape(-1)
    t = np.ascontiguousarray(np.asarray(targets, dtype=np.int32).reshape(-1))
    rows = t.size
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32).reshape(-1)
    loss = np.zeros(1, dtype=np.float32)
    hg = np.zeros(rows * w.rows, dtype=np.float32) if grads else None
    bg = np.zeros(w.columns, dtype=np.float32) if grads else None
    st = lib().ko_fused_cross_entropy(_p(hidden), rows, ctypes.byref(w.qw), _p(b), _p(t), ignore_index, _p(loss),
                                      _p(hg), _p(bg), threads)
    if st != KO_OK:
        raise ValueError(f"oracle fused_cross_entropy status {st}")
    return float(loss[0]), (None if hg is None else hg.reshape(rows, w.rows)), bg


def multiply_by_quantized_transposed(dy: np.ndarray, w: Quantized, m: int, dx: np.ndarray | None = None,
                                     accumulate: bool = False, threads: int = 1) -> np.ndarray:
    dy = np.ascontiguousarray(dy, dtype=np.float32).reshape(-1)
    if dx is None:
        dx = np.zeros(m * w.rows, dtype=np.float32)
    dx = np.ascontiguousarray(dx, dtype=np.float32).reshape(-1).copy()
    st = lib().ko_multiply_by_quantized_transposed(_p(dy), ctypes.byref(w.qw), _p(dx), m, int(accumulate), threads)
    if st != KO_OK:
        raise ValueError(f"oracle transposed status {st}")
    return dx.reshape(m, w.rows)


# ---- decoder pieces (kt_oracle_decoder.c) ------------------------------------------


def rope_inv_freq(head_dim: int, base: float, scaling: tuple | None = None) -> np.ndarray:
    """RoPE.invFreq; scaling = (factor, low, high, original_max) or None."""
    out = np.empty(head_dim // 2, dtype=np.float32)
    f, lo, hi, om = scaling if scaling else (0.0, 1.0, 4.0, 8192)
    lib().ko_rope_inv_freq(head_dim, ctypes.c_float(base), ctypes.c_float(f), ctypes.c_float(lo), ctypes.c_float(hi),
                           int(om), _p(out))
    return out


def rmsnorm(x: np.ndarray, weight: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, dim = x.reshape(-1, weight.size).shape
    out = np.empty_like(x)
    lib().ko_rmsnorm(_p(x), rows, dim, _p(np.ascontiguousarray(weight, dtype=np.float32)), ctypes.c_float(eps), _p(out))
    return out


def rope_rows(rows: np.ndarray, head_dim: int, inv_freq: np.ndarray, start: int) -> np.ndarray:
    """A rotated copy of rows [tokens x width]."""
    out = np.array(rows, dtype=np.float32, copy=True, order="C")
    tokens, width = out.shape
    lib().ko_rope_rows(_p(out), tokens, width, head_dim, _p(np.ascontiguousarray(inv_freq, dtype=np.float32)), start)
    return out


def attend(q: np.ndarray, start: int, keys: np.ndarray, values: np.ndarray, layer: int, num_heads: int,
           num_kv_heads: int, head_dim: int, max_seq: int) -> np.ndarray:
    """attendCached for q [tokens x num_heads*head_dim] over caches in the KVCache layout."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    tokens = q.shape[0]
    context = np.empty_like(q)
    scores = np.empty(start + tokens, dtype=np.float32)
    lib().ko_attend(_p(q), tokens, start, _p(keys), _p(values), layer, num_heads, num_kv_heads, head_dim, max_seq,
                    _p(context), _p(scores))
    return context


def silu_mul(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    out = np.array(gate, dtype=np.float32, copy=True, order="C")
    lib().ko_silu_mul(_p(out), _p(np.ascontiguousarray(up, dtype=np.float32)), out.size)
    return out


def argmax(logits: np.ndarray) -> int:
    x = np.ascontiguousarray(logits, dtype=np.float32).reshape(-1)
    return int(lib().ko_argmax(_p(x), x.size))
