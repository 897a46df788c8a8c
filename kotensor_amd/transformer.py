"""The quantized decoder, device-resident: ``Transformer``, ``KVCache`` and
``InferenceBuffers``.

Mirrors the reference's inference path (Engine/kotensor/src/main/kotlin/):
``Transformer.newCache / newInferenceBuffers / prefill / decode / generate``
(Transformer.kt:76-233), ``TransformerBlock.decodeInto / prefillInto``
(TransformerBlock.kt:204-220), ``Attention.decodeInto / prefillInto``
(Attention.kt:207-275), ``SwiGLU.forwardInto`` (SwiGLU.kt:19-25), ``KVCache``
(KVCache.kt:3-59), ``InferenceBuffers`` (InferenceBuffers.kt:3-53) and
``saveQuantized / loadQuantized`` (Transformer.kt:402-471), with the reference's names,
argument checks and messages. Every projection is a quantized GEMV/GEMM of
libkotensor_hip.so and every other step a kernel of kt_decoder.hip; the activations,
the KV cache and its length stay on the device, so ``generate`` can record one decode
step as a HIP graph and replay it per token.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from .device import DeviceBuffer, Stream, default_stream
from .quantization import Quantization, QuantizedTensor

TILE_M = 32  # MatMul.TILE_M (MatMul.kt:16), the reference's prefill chunk


def _stream(stream: Stream | None):
    return (stream or default_stream()).handle


def java_float_string(v: float) -> str:
    """Float.toString: the shortest decimal that reads back as the same float, plain for
    1e-3 <= |v| < 1e7 ("10000.0", "0.02"), else "d.dddE<exp>" ("1.0E-6", "1.0E7")."""
    f = np.float32(v)
    if f == 0:
        return "-0.0" if np.signbit(f) else "0.0"
    if not np.isfinite(f):
        return "NaN" if np.isnan(f) else ("Infinity" if f > 0 else "-Infinity")
    if 1e-3 <= abs(float(f)) < 1e7:
        return np.format_float_positional(f, unique=True, trim="0")
    s = np.format_float_scientific(f, unique=True, trim="0", exp_digits=1)
    mant, exp = s.split("e")
    return f"{mant}E{int(exp)}"


class RoPEScaling:
    """RoPEScaling (RoPE.kt:7-31)."""

    def __init__(self, factor: float, low_frequency_factor: float = 1.0, high_frequency_factor: float = 4.0,
                 original_max_position_embeddings: int = 8192):
        if not (factor > 0 and original_max_position_embeddings > 0):
            raise _lib.IllegalArgumentException("Invalid RoPE scaling")
        if not high_frequency_factor > low_frequency_factor:
            raise _lib.IllegalArgumentException("highFrequencyFactor must exceed lowFrequencyFactor")
        self.factor = float(factor)
        self.low_frequency_factor = float(low_frequency_factor)
        self.high_frequency_factor = float(high_frequency_factor)
        self.original_max_position_embeddings = int(original_max_position_embeddings)

    def as_tuple(self):
        return (self.factor, self.low_frequency_factor, self.high_frequency_factor,
                self.original_max_position_embeddings)


def rope_inv_freq(head_dim: int, base: float, scaling: RoPEScaling | None = None) -> np.ndarray:
    """RoPE.invFreq (RoPE.kt:42-46), computed by the library on the host."""
    out = np.empty(head_dim // 2, dtype=np.float32)
    f, lo, hi, om = scaling.as_tuple() if scaling else (0.0, 1.0, 4.0, 8192)
    _lib.call("kt_rope_inv_freq", head_dim, ctypes.c_float(base), ctypes.c_float(f), ctypes.c_float(lo),
              ctypes.c_float(hi), int(om), out.ctypes.data_as(ctypes.c_void_p))
    return out


class KVCache:
    """KVCache (KVCache.kt:3-59) in device memory: keys and values of
    ``[layers x heads x max_sequence_length x head_dim]`` fp32 and the length, kept on
    the host and, for the kernels, as a device int32."""

    def __init__(self, num_layers: int, num_heads: int, max_sequence_length: int, head_dim: int,
                 stream: Stream | None = None):
        if num_layers <= 0:
            raise _lib.IllegalArgumentException("numLayers must be positive")
        if num_heads <= 0:
            raise _lib.IllegalArgumentException("numHeads must be positive")
        if max_sequence_length <= 0:
            raise _lib.IllegalArgumentException("maxSequenceLength must be positive")
        if head_dim <= 0:
            raise _lib.IllegalArgumentException("headDim must be positive")
        self.num_layers, self.num_heads = int(num_layers), int(num_heads)
        self.max_sequence_length, self.head_dim = int(max_sequence_length), int(head_dim)
        n = self.num_layers * self.num_heads * self.max_sequence_length * self.head_dim
        self.keys = DeviceBuffer(n * 4)
        self.values = DeviceBuffer(n * 4)
        self.position = DeviceBuffer(4)
        for b in (self.keys, self.values, self.position):
            b.fill_zero(stream)
        self.length = 0

    @property
    def remaining(self) -> int:
        return self.max_sequence_length - self.length

    def offset(self, layer: int, head: int, position: int) -> int:
        return ((layer * self.num_heads + head) * self.max_sequence_length + position) * self.head_dim

    def check_room(self, count: int) -> None:
        if count < 0:
            raise _lib.IllegalArgumentException("count must not be negative")
        if self.length + count > self.max_sequence_length:
            raise _lib.IllegalArgumentException(
                f"KV cache full: {self.length} + {count} positions exceed maxSequenceLength {self.max_sequence_length}")

    def advance(self, count: int, stream: Stream | None = None) -> None:
        """KVCache.advance: the host length and the device length move together."""
        self.check_room(count)
        _lib.call("kt_position_add", self.position.ptr, int(count), _stream(stream))
        self.length += count

    def reset(self, stream: Stream | None = None) -> None:
        self.position.fill_zero(stream)
        self.length = 0

    def copy_from(self, source: "KVCache", length: int, stream: Stream | None = None) -> None:
        """KVCache.copyFrom (KVCache.kt:41-55)."""
        if (source.num_layers, source.num_heads, source.head_dim) != (self.num_layers, self.num_heads, self.head_dim):
            raise _lib.IllegalArgumentException(
                f"Cannot copy a cache of {source.num_layers} layers × {source.num_heads} heads × {source.head_dim} dims "
                f"into {self.num_layers} × {self.num_heads} × {self.head_dim}")
        if not 0 <= length <= source.length:
            raise _lib.IllegalArgumentException(f"Cannot copy {length} positions from a cache holding {source.length}")
        if length > self.max_sequence_length:
            raise _lib.IllegalArgumentException(f"Cannot copy {length} positions into a cache of {self.max_sequence_length}")
        count = length * self.head_dim * 4
        st = _stream(stream)
        for layer in range(self.num_layers):
            for head in range(self.num_heads):
                for dst, src in ((self.keys, source.keys), (self.values, source.values)):
                    if count:
                        _lib.call("kt_memcpy_d2d", dst.ptr + self.offset(layer, head, 0) * 4,
                                  src.ptr + source.offset(layer, head, 0) * 4, ctypes.c_size_t(count), st)
        self.position.upload(np.array([length], np.int32), stream)
        self.length = length

    @property
    def size_in_bytes(self) -> int:
        return self.keys.nbytes + self.values.nbytes

    def keys_numpy(self, stream: Stream | None = None) -> np.ndarray:
        return self.keys.download(np.float32, stream=stream)

    def values_numpy(self, stream: Stream | None = None) -> np.ndarray:
        return self.values.download(np.float32, stream=stream)


class _Rows:
    """The activations of ``rows`` tokens (InferenceBuffers / PrefillBuffers,
    InferenceBuffers.kt:3-53)."""

    def __init__(self, rows: int, dimension: int, hidden_dimension: int, kv_dimension: int):
        self.rows = rows
        f = 4
        self.tokens = DeviceBuffer(4 * rows)
        self.x = DeviceBuffer(rows * dimension * f)
        self.normed = DeviceBuffer(rows * dimension * f)
        self.q = DeviceBuffer(rows * dimension * f)
        self.k = DeviceBuffer(rows * kv_dimension * f)
        self.v = DeviceBuffer(rows * kv_dimension * f)
        self.context = DeviceBuffer(rows * dimension * f)
        self.attention_out = DeviceBuffer(rows * dimension * f)
        self.gate = DeviceBuffer(rows * hidden_dimension * f)
        self.up = DeviceBuffer(rows * hidden_dimension * f)
        self.ffn_out = DeviceBuffer(rows * dimension * f)


class InferenceBuffers(_Rows):
    """InferenceBuffers (InferenceBuffers.kt:3-32): one token's activations, the logits
    and the greedy token, all on the device, plus prefill buffers made on demand."""

    def __init__(self, dimension: int, hidden_dimension: int, vocabulary_size: int, max_sequence_length: int,
                 kv_dimension: int | None = None):
        kv_dimension = dimension if kv_dimension is None else kv_dimension
        if min(dimension, hidden_dimension, vocabulary_size, max_sequence_length, kv_dimension) <= 0:
            raise _lib.IllegalArgumentException("InferenceBuffers dimensions must be positive")
        super().__init__(1, dimension, hidden_dimension, kv_dimension)
        self.dimension, self.hidden_dimension = dimension, hidden_dimension
        self.vocabulary_size, self.max_sequence_length, self.kv_dimension = vocabulary_size, max_sequence_length, kv_dimension
        self.logits = DeviceBuffer(vocabulary_size * 4)
        self.generated = DeviceBuffer(4 * max_sequence_length)  # greedy tokens by position
        self._prefill: dict[int, _Rows] = {}

    def prefill_rows(self, rows: int) -> _Rows:
        if rows not in self._prefill:
            self._prefill.clear()
            self._prefill[rows] = _Rows(rows, self.dimension, self.hidden_dimension, self.kv_dimension)
        return self._prefill[rows]

    def logits_numpy(self, stream: Stream | None = None) -> np.ndarray:
        return self.logits.download(np.float32, stream=stream)

    @property
    def size_in_bytes(self) -> int:
        return (6 * self.dimension + 2 * self.kv_dimension + 2 * self.hidden_dimension + self.vocabulary_size) * 4


def _group(weights: list[QuantizedTensor], outs: list[int], biases: list[int | None]):
    n = len(weights)
    ws = (_lib.QWeight * n)(*[w.qweight for w in weights])
    os_ = (ctypes.c_void_p * n)(*outs)
    bs = None if all(b is None for b in biases) else (ctypes.c_void_p * n)(*[b or 0 for b in biases])
    return n, ws, os_, bs


class Transformer:
    """The quantized Transformer (Transformer.kt:3-22) on the device.

    Weights follow the reference's names (Transformer.kt:268-359): the quantized
    ``embedding`` table (absent when tied to the head), ``block.{l}.attention.wQ/wK/wV/wOut``,
    ``block.{l}.ffn.wGate/wUp/wDown`` and ``lmHead`` (QuantizedTensor ``[in x out]``), and
    the fp32 parameters ``block.{l}.norm1.weight``, ``block.{l}.norm2.weight``,
    ``finalNorm.weight`` and ``{projection}.bias``.
    """

    def __init__(self, vocabulary_size: int, dimension: int, num_layers: int, num_heads: int,
                 hidden_dimension: int | None = None, num_key_value_heads: int | None = None,
                 norm_eps: float = 1e-6, rope_theta: float = 10000.0, rope_scaling: RoPEScaling | None = None,
                 quantization: Quantization | None = None, seed: int | None = 0, init_std: float = 0.02,
                 stream: Stream | None = None, packed: bool = True):
        hidden_dimension = 4 * dimension if hidden_dimension is None else hidden_dimension
        num_key_value_heads = num_heads if num_key_value_heads is None else num_key_value_heads
        if dimension % num_heads != 0:
            raise _lib.IllegalArgumentException("dimension must be divisible by numHeads")
        if not (1 <= num_key_value_heads <= num_heads and num_heads % num_key_value_heads == 0):
            raise _lib.IllegalArgumentException(
                f"numHeads {num_heads} must be a multiple of numKeyValueHeads {num_key_value_heads}")
        if (dimension // num_heads) % 2 != 0:
            raise _lib.IllegalArgumentException("RoPE dimension must be even")
        self.vocabulary_size, self.dimension, self.num_layers = vocabulary_size, dimension, num_layers
        self.num_heads, self.hidden_dimension, self.num_key_value_heads = num_heads, hidden_dimension, num_key_value_heads
        self.norm_eps, self.rope_theta, self.rope_scaling = float(norm_eps), float(rope_theta), rope_scaling
        self.quantization = quantization or Quantization.INT4
        self.head_dim = dimension // num_heads
        self.kv_dimension = num_key_value_heads * self.head_dim
        self.tied = False
        self.inv_freq = DeviceBuffer.from_numpy(rope_inv_freq(self.head_dim, self.rope_theta, rope_scaling), stream)
        self.weights: dict[str, QuantizedTensor] = {}
        self.parameters: dict[str, DeviceBuffer] = {}
        self._zero_bias: dict[str, bool] = {}
        for name, (k, n) in self.projection_shapes().items():
            self.weights[name] = (self._random_weight(k, n, seed, init_std, len(self.weights), stream)
                                  if seed is not None else QuantizedTensor.empty(k, n, self.quantization))
            self.set_parameter(f"{name}.bias", np.zeros(n, np.float32), stream)
        self.weights["embedding"] = (self._random_weight(vocabulary_size, dimension, seed, init_std, len(self.weights),
                                                         stream)
                                     if seed is not None else QuantizedTensor.empty(vocabulary_size, dimension,
                                                                                    self.quantization))
        for l in range(num_layers):
            self.set_parameter(f"block.{l}.norm1.weight", np.ones(dimension, np.float32), stream)
            self.set_parameter(f"block.{l}.norm2.weight", np.ones(dimension, np.float32), stream)
        self.set_parameter("finalNorm.weight", np.ones(dimension, np.float32), stream)
        self._graph = None
        # one-row steps: the projections between two attention calls as one chained launch
        # (kt_qmatmul_chain) when True, else as separate launches (the default: at the
        # 1B decoder's shapes measured 0.488 ms per token separate, 0.538 chained)
        self.chain_one_row = False
        # column-run copies of the projections for the one-row (decode) products
        self.packed = packed
        if packed and seed is not None:
            self.pack_weights(stream)

    def pack_weights(self, stream: Stream | None = None) -> None:
        """Writes the column-run copy of every projection weight (QuantizedTensor.pack), which
        the decode step's one-row products read, and the prefill GEMM too when the group
        size is a multiple of 32."""
        for name in self.projection_shapes():
            self.weights[name].pack(stream)
        self.packed = True

    # -- construction --------------------------------------------------------------------
    def projection_shapes(self) -> dict:
        """namedProjections (Transformer.kt:268-282) with their ``[in x out]`` shapes."""
        d, kv, h = self.dimension, self.kv_dimension, self.hidden_dimension
        out = {}
        for l in range(self.num_layers):
            p = f"block.{l}."
            out[p + "attention.wQ"] = (d, d)
            out[p + "attention.wK"] = (d, kv)
            out[p + "attention.wV"] = (d, kv)
            out[p + "attention.wOut"] = (d, d)
            out[p + "ffn.wGate"] = (d, h)
            out[p + "ffn.wUp"] = (d, h)
            out[p + "ffn.wDown"] = (h, d)
        out["lmHead"] = (d, self.vocabulary_size)
        return out

    def _random_weight(self, k: int, n: int, seed: int, std: float, index: int, stream) -> QuantizedTensor:
        buf = DeviceBuffer(k * n * 4)
        _lib.call("kt_fill_normal", buf.ptr, ctypes.c_int64(k * n), ctypes.c_uint64((seed * 1000003 + index) & (2**64 - 1)),
                  ctypes.c_float(0.0), ctypes.c_float(std), _stream(stream))
        w = QuantizedTensor.quantize(buf, k, n, self.quantization, stream)
        buf.free()
        return w

    def set_parameter(self, name: str, value, stream: Stream | None = None) -> None:
        arr = np.ascontiguousarray(value, dtype=np.float32).reshape(-1)
        self.parameters[name] = DeviceBuffer.from_numpy(arr, stream)
        if name.endswith(".bias"):
            self._zero_bias[name[:-5]] = not np.any(arr)

    def set_weight(self, name: str, weight: QuantizedTensor) -> None:
        if name == "embedding":
            want = (self.vocabulary_size, self.dimension)
        else:
            want = self.projection_shapes()[name]
        if (weight.rows, weight.columns) != want:
            raise _lib.IllegalArgumentException(
                f"Quantized weight is {weight.rows} × {weight.columns}, layer is {want[0]} × {want[1]}")
        if self.packed and name != "embedding":
            weight.pack()
        self.weights[name] = weight

    def tie_embedding_to_head(self) -> "Transformer":
        """tieEmbeddingToHead (Transformer.kt:380-386): tokens read head columns."""
        self.tied = True
        self.weights.pop("embedding", None)
        return self

    @property
    def is_embedding_tied(self) -> bool:
        return self.tied

    # -- saveQuantized / loadQuantized -----------------------------------------------------
    def metadata(self) -> dict:
        """The kotensor.* keys saveQuantized writes (Transformer.kt:404-419)."""
        def jfloat(v: float) -> str:
            return java_float_string(v)
        meta = {"kotensor.vocabularySize": str(self.vocabulary_size), "kotensor.dimension": str(self.dimension),
                "kotensor.numLayers": str(self.num_layers), "kotensor.numHeads": str(self.num_heads),
                "kotensor.hiddenDimension": str(self.hidden_dimension),
                "kotensor.numKeyValueHeads": str(self.num_key_value_heads),
                "kotensor.normEps": jfloat(self.norm_eps), "kotensor.ropeTheta": jfloat(self.rope_theta)}
        if self.rope_scaling:
            s = self.rope_scaling
            meta["kotensor.ropeScaling"] = (f"{jfloat(s.factor)},{jfloat(s.low_frequency_factor)},"
                                            f"{jfloat(s.high_frequency_factor)},{s.original_max_position_embeddings}")
        meta["kotensor.quantization.bits"] = str(self.quantization.bits)
        meta["kotensor.quantization.groupSize"] = str(self.quantization.group_size)
        if self.tied:
            meta["kotensor.tiedEmbedding"] = "true"
        return meta

    def save_quantized(self, path, stream: Stream | None = None) -> None:
        """saveQuantized (Transformer.kt:402-430): the fp32 parameters, then each quantized
        weight's .qweight / .scales / .zeros straight from device memory."""
        from .safetensors import save_quantized
        params = {name: buf.download(np.float32, stream=stream) for name, buf in self.parameters.items()}
        order = ([] if self.tied else ["embedding"]) + list(self.projection_shapes())
        save_quantized(path, params, {n: self.weights[n] for n in order}, self.metadata(), stream)

    @classmethod
    def load_quantized(cls, path, stream: Stream | None = None) -> "Transformer":
        """loadQuantized (Transformer.kt:432-471): the configuration from the kotensor.*
        metadata, the quantized weights copied from the mapped file into device buffers."""
        from .safetensors import SafeTensorsFile
        with SafeTensorsFile(path) as f:
            meta = f.metadata

            def value(key: str) -> str:
                if key not in meta:
                    raise _lib.IllegalArgumentException(f"{path} has no {key} metadata; was it written by saveQuantized?")
                return meta[key]
            scaling = None
            if "kotensor.ropeScaling" in meta:
                p = meta["kotensor.ropeScaling"].split(",")
                scaling = RoPEScaling(float(p[0]), float(p[1]), float(p[2]), int(p[3]))
            q = Quantization(int(value("kotensor.quantization.bits")), int(value("kotensor.quantization.groupSize")))
            model = cls(int(value("kotensor.vocabularySize")), int(value("kotensor.dimension")),
                        int(value("kotensor.numLayers")), int(value("kotensor.numHeads")),
                        int(value("kotensor.hiddenDimension")), int(value("kotensor.numKeyValueHeads")),
                        float(value("kotensor.normEps")), float(value("kotensor.ropeTheta")), scaling, q, seed=None,
                        stream=stream)
            if meta.get("kotensor.tiedEmbedding") == "true":
                model.tie_embedding_to_head()
            for name in list(model.parameters):
                if name not in f:
                    raise _lib.IllegalArgumentException(f"{path} is missing {name}")
                model.set_parameter(name, f.load(name), stream)
            for name in list(model.weights):
                k, n = (model.vocabulary_size, model.dimension) if name == "embedding" else model.projection_shapes()[name]
                model.weights[name] = f.load_quantized(name, q, k, n, stream)
            if model.packed:
                model.pack_weights(stream)
            return model

    # -- caches and buffers -------------------------------------------------------------
    def new_cache(self, max_sequence_length: int, stream: Stream | None = None) -> KVCache:
        return KVCache(self.num_layers, self.num_key_value_heads, max_sequence_length, self.head_dim, stream)

    def new_inference_buffers(self, max_sequence_length: int) -> InferenceBuffers:
        return InferenceBuffers(self.dimension, self.hidden_dimension, self.vocabulary_size, max_sequence_length,
                                self.kv_dimension)

    def _check(self, cache: KVCache, buffers: InferenceBuffers, count: int) -> None:
        if cache.num_layers != self.num_layers:
            raise _lib.IllegalArgumentException(f"Cache built for {cache.num_layers} layers, model has {self.num_layers}")
        if cache.remaining < count:
            raise _lib.IllegalArgumentException(
                f"KV cache full: {cache.length} + {count} positions exceed maxSequenceLength {cache.max_sequence_length}")
        if (buffers.dimension, buffers.hidden_dimension, buffers.vocabulary_size, buffers.kv_dimension) != \
                (self.dimension, self.hidden_dimension, self.vocabulary_size, self.kv_dimension):
            raise _lib.IllegalArgumentException("InferenceBuffers built for another model configuration")
        if buffers.max_sequence_length < cache.length + count:
            raise _lib.IllegalArgumentException(
                f"InferenceBuffers sized for {buffers.max_sequence_length} positions, prompt ends at {cache.length + count}")

    # -- the step ---------------------------------------------------------------------
    def _embed(self, rows: _Rows, count: int, st) -> None:
        if self.tied:
            _lib.call("kt_dequantize_columns", ctypes.byref(self.weights["lmHead"].qweight), rows.tokens.ptr, count,
                      rows.x.ptr, st)
        else:
            _lib.call("kt_dequantize_rows", ctypes.byref(self.weights["embedding"].qweight), rows.tokens.ptr, count,
                      rows.x.ptr, st)

    def _residual_projection(self, name: str, a: DeviceBuffer, rows: _Rows, count: int, st) -> None:
        """x += a · deq(W) + bias, rounded as Tensor.addInPlace after forwardInto: a zero
        bias lets the product accumulate straight into x."""
        w = self.weights[name]
        if self._zero_bias.get(name, True):
            _lib.call("kt_qmatmul", a.ptr, count, ctypes.byref(w.qweight), rows.x.ptr, 1, ctypes.c_float(1.0), st)
        else:
            _lib.call("kt_qlinear_forward", a.ptr, count, ctypes.byref(w.qweight), self.parameters[name + ".bias"].ptr,
                      rows.attention_out.ptr, st)
            _lib.call("kt_add_inplace", rows.x.ptr, rows.attention_out.ptr, ctypes.c_int64(count * self.dimension), st)

    def _bias(self, name: str):
        return None if self._zero_bias.get(name, True) else self.parameters[name + ".bias"].ptr

    def _layers(self, rows: _Rows, count: int, cache: KVCache, key_bound: int, st,
                head: InferenceBuffers | None = None) -> bool:
        """The layers over `count` rows. For one row the projections between two attention
        calls (wOut, norm2 and the gate pair, wDown, and the next layer's norm1 and q/k/v)
        run as one kt_qmatmul_chain call, and with `head` the last layer's chain ends with
        finalNorm and lmHead into head.logits; returns whether the head ran."""
        q_ready = False  # the layer's q/k/v came from the previous layer's chain
        headed = False
        for l in range(self.num_layers):
            p = f"block.{l}."
            if not q_ready:
                n, ws, os_, bs = _group([self.weights[x] for x in self._qkv_names(l)], [rows.q.ptr, rows.k.ptr, rows.v.ptr],
                                        [self._bias(x) for x in self._qkv_names(l)])
                _lib.call("kt_rmsnorm_qmatmul_group", rows.x.ptr, self.parameters[p + "norm1.weight"].ptr,
                          ctypes.c_float(self.norm_eps), rows.normed.ptr, count, ws, n, os_, bs, 0, ctypes.c_float(1.0),
                          st)
            _lib.call("kt_rope_attention", rows.q.ptr, rows.k.ptr, rows.v.ptr, self.inv_freq.ptr, count,
                      cache.position.ptr, key_bound, cache.keys.ptr, cache.values.ptr, l, cache.max_sequence_length,
                      self.num_heads, self.num_key_value_heads, self.head_dim, rows.context.ptr, st)
            q_ready = False
            if count == 1 and self.chain_one_row and self._zero_bias.get(p + "attention.wOut", True) and \
                    self._zero_bias.get(p + "ffn.wDown", True):
                # a zero bias lets wOut and wDown accumulate straight into x
                steps = [(rows.context.ptr, None, [self.weights[p + "attention.wOut"]], [rows.x.ptr], [None], 1, 0),
                         (rows.x.ptr, self.parameters[p + "norm2.weight"].ptr,
                          [self.weights[p + "ffn.wGate"], self.weights[p + "ffn.wUp"]], [rows.gate.ptr, rows.up.ptr],
                          [self._bias(p + "ffn.wGate"), self._bias(p + "ffn.wUp")], 0, 1),
                         (rows.gate.ptr, None, [self.weights[p + "ffn.wDown"]], [rows.x.ptr], [None], 1, 0)]
                if l + 1 < self.num_layers:
                    names = self._qkv_names(l + 1)
                    steps.append((rows.x.ptr, self.parameters[f"block.{l + 1}.norm1.weight"].ptr,
                                  [self.weights[x] for x in names], [rows.q.ptr, rows.k.ptr, rows.v.ptr],
                                  [self._bias(x) for x in names], 0, 0))
                    q_ready = True
                elif head is not None:
                    steps.append((rows.x.ptr, self.parameters["finalNorm.weight"].ptr, [self.weights["lmHead"]],
                                  [head.logits.ptr], [self._bias("lmHead")], 0, 0))
                    headed = True
                self._chain(steps, rows.normed.ptr, st)
                continue
            self._residual_projection(p + "attention.wOut", rows.context, rows, count, st)
            # norm2, gate and up, and the gate silu(gate) * up in one call; then the down
            # projection of the gate row with the residual
            _lib.call("kt_rmsnorm_swiglu_gate", rows.x.ptr, self.parameters[p + "norm2.weight"].ptr,
                      ctypes.c_float(self.norm_eps), rows.normed.ptr, count,
                      ctypes.byref(self.weights[p + "ffn.wGate"].qweight), ctypes.byref(self.weights[p + "ffn.wUp"].qweight),
                      self._bias(p + "ffn.wGate"), self._bias(p + "ffn.wUp"), rows.gate.ptr, rows.up.ptr, st)
            self._residual_projection(p + "ffn.wDown", rows.gate, rows, count, st)
        return headed

    @staticmethod
    def _qkv_names(l: int) -> list[str]:
        p = f"block.{l}."
        return [p + "attention.wQ", p + "attention.wK", p + "attention.wV"]

    def _chain(self, steps, normed_ptr: int, st) -> None:
        """kt_qmatmul_chain over (x, norm weight, weights, outputs, biases, accumulate,
        swiglu gate pair) steps."""
        arr = (_lib.QMatmulStep * len(steps))()
        keep = []
        for s, (x, nw, ws, outs, biases, acc, swiglu) in zip(arr, steps):
            n = len(ws)
            wa = (_lib.QWeight * n)(*[w.qweight for w in ws])
            oa = (ctypes.c_void_p * n)(*outs)
            ba = None if all(b is None for b in biases) else (ctypes.c_void_p * n)(*[b or 0 for b in biases])
            keep += [wa, oa, ba]
            s.x, s.norm_weight, s.eps, s.normed = x, nw, self.norm_eps, normed_ptr
            s.weights = ctypes.cast(wa, ctypes.POINTER(_lib.QWeight))
            s.count = n
            s.outputs = ctypes.cast(oa, ctypes.POINTER(ctypes.c_void_p))
            s.biases = ctypes.cast(ba, ctypes.POINTER(ctypes.c_void_p)) if ba is not None else None
            s.accumulate, s.alpha, s.swiglu_gate = acc, 1.0, swiglu
        _lib.call("kt_qmatmul_chain", arr, len(steps), st)

    def _head(self, x_row_ptr: int, buffers: InferenceBuffers, st) -> None:
        """finalNorm and lmHead of one row into buffers.logits (one launch with the norm
        inside the product where the one-row kernels take it)."""
        n, ws, os_, bs = _group([self.weights["lmHead"]], [buffers.logits.ptr], [self._bias("lmHead")])
        _lib.call("kt_rmsnorm_qmatmul_group", x_row_ptr, self.parameters["finalNorm.weight"].ptr,
                  ctypes.c_float(self.norm_eps), buffers.normed.ptr, 1, ws, n, os_, bs, 0, ctypes.c_float(1.0), st)

    def _decode_step(self, cache: KVCache, buffers: InferenceBuffers, st, argmax: bool) -> None:
        """One token from buffers.tokens[0] at the device position; the host length is the
        caller's to advance. With argmax the greedy token replaces buffers.tokens[0] and is
        recorded in buffers.generated at its position."""
        self._embed(buffers, 1, st)
        headed = self._layers(buffers, 1, cache, cache.max_sequence_length, st, head=buffers)
        if not headed:
            self._head(buffers.x.ptr, buffers, st)
        if argmax:
            # the head does not read the position: advance it, take the argmax and record
            # the token in one launch after the head
            _lib.call("kt_argmax_advance", buffers.logits.ptr, self.vocabulary_size, buffers.tokens.ptr,
                      cache.position.ptr, buffers.generated.ptr, buffers.max_sequence_length, st)
        else:
            _lib.call("kt_position_add", cache.position.ptr, 1, st)

    # -- the reference's entry points ----------------------------------------------------
    def prefill(self, prompt, cache: KVCache, buffers: InferenceBuffers, stream: Stream | None = None,
                chunk_rows: int | None = None) -> InferenceBuffers:
        """Transformer.prefill (Transformer.kt:99-132): every layer over the prompt in
        chunks (by default one chunk: the GPU takes the whole prompt as one GEMM; the
        reference uses 32 rows), then finalNorm and lmHead on the last row into
        buffers.logits. Returns the buffers (logits via buffers.logits_numpy())."""
        prompt = [int(t) for t in prompt]
        if not prompt:
            raise _lib.IllegalArgumentException("Prompt cannot be empty")
        self._check(cache, buffers, len(prompt))
        for t in prompt:
            if not 0 <= t < self.vocabulary_size:
                raise _lib.IllegalArgumentException(f"{t} out of vocab bounds {self.vocabulary_size}")
        st = _stream(stream)
        chunk = chunk_rows or len(prompt)
        rows = None
        for start in range(0, len(prompt), chunk):
            part = prompt[start:start + chunk]
            rows = buffers.prefill_rows(len(part))
            rows.tokens.upload(np.array(part, np.int32), stream)
            self._embed(rows, len(part), st)
            self._layers(rows, len(part), cache, cache.length + len(part), st)
            cache.advance(len(part), stream)
        self._head(rows.x.ptr + (rows.rows - 1) * self.dimension * 4, buffers, st)
        return buffers

    def decode(self, token: int, cache: KVCache, buffers: InferenceBuffers,
               stream: Stream | None = None) -> InferenceBuffers:
        """Transformer.decode (Transformer.kt:141-154)."""
        if cache.num_layers != self.num_layers:
            raise _lib.IllegalArgumentException(f"Cache built for {cache.num_layers} layers, model has {self.num_layers}")
        if cache.remaining < 1:
            raise _lib.IllegalArgumentException(f"KV cache full: maxSequenceLength {cache.max_sequence_length}")
        self._check(cache, buffers, 1)
        if not 0 <= int(token) < self.vocabulary_size:
            raise _lib.IllegalArgumentException(f"{token} out of vocab bounds {self.vocabulary_size}")
        buffers.tokens.upload(np.array([int(token)], np.int32), stream)
        self._decode_step(cache, buffers, _stream(stream), argmax=False)
        cache.length += 1
        return buffers

    def greedy_decode(self, cache: KVCache, buffers: InferenceBuffers, steps: int, stream: Stream | None = None,
                      use_graph: bool = True) -> list[int]:
        """The greedy part of streamFrom (Transformer.kt:224-231) after a prefill: takes
        the argmax of buffers.logits, then `steps` decode steps, each feeding the previous
        greedy token (which never leaves the device) and taking the next argmax. Returns
        the steps + 1 greedy tokens. With use_graph (on a created, non-null stream) one
        decode step is recorded as a HIP graph and replayed."""
        if cache.remaining < steps:
            raise _lib.IllegalArgumentException(
                f"KV cache full: {cache.length} + {steps} positions exceed maxSequenceLength {cache.max_sequence_length}")
        if buffers.max_sequence_length < cache.length + steps + 1:
            raise _lib.IllegalArgumentException(
                f"InferenceBuffers sized for {buffers.max_sequence_length} positions, generation ends at "
                f"{cache.length + steps + 1}")
        st = _stream(stream)
        first = cache.length
        _lib.call("kt_argmax", buffers.logits.ptr, self.vocabulary_size, buffers.tokens.ptr, st)
        _lib.call("kt_record_token", buffers.tokens.ptr, cache.position.ptr, buffers.generated.ptr,
                  buffers.max_sequence_length, st)
        if use_graph and steps > 1 and st:
            self.decode_step(cache, buffers, stream)  # the first step also sizes the workspaces
            graph = self.capture_decode(cache, buffers, stream)
            try:
                graph.replay(steps - 1)
            finally:
                (stream or default_stream()).synchronize()
                graph.destroy()
        else:
            for _ in range(steps):
                self.decode_step(cache, buffers, stream)
        return buffers.generated.download(np.int32, count=steps + 1, stream=stream, offset=4 * first).tolist()

    def decode_step(self, cache: KVCache, buffers: InferenceBuffers, stream: Stream | None = None) -> None:
        """One greedy decode step on the device: the token in buffers.tokens (the last
        argmax) in, its logits in buffers.logits, the next argmax in buffers.tokens and in
        buffers.generated at its position."""
        cache.check_room(1)
        self._decode_step(cache, buffers, _stream(stream), argmax=True)
        cache.length += 1

    def capture_decode(self, cache: KVCache, buffers: InferenceBuffers, stream: Stream) -> "DecodeGraph":
        """decode_step recorded once as a HIP graph on `stream` (a created stream; run one
        decode_step first so the library's workspaces already have their sizes)."""
        st = _stream(stream)
        if not st:
            raise _lib.IllegalArgumentException("the null stream cannot be captured; create a stream")
        _lib.call("kt_graph_begin", st)
        graph = ctypes.c_void_p()
        try:
            self._decode_step(cache, buffers, st, argmax=True)
        except BaseException:
            # end the capture so the stream is usable again, and drop the partial graph
            if _lib.lib().kt_graph_end(st, ctypes.byref(graph)) == _lib.KT_OK and graph:
                _lib.lib().kt_graph_destroy(graph)
            raise
        _lib.call("kt_graph_end", st, ctypes.byref(graph))
        return DecodeGraph(graph, cache, stream)

    def generate(self, prompt, max_tokens: int, stop_tokens=(), stream: Stream | None = None,
                 use_graph: bool = True) -> list[int]:
        """Greedy generate (Transformer.kt:167-233): prefill, then argmax and decode,
        stopping at a stop token. The greedy token never leaves the device between steps;
        with use_graph one decode step is recorded as a HIP graph and replayed."""
        prompt = [int(t) for t in prompt]
        if not prompt:
            raise _lib.IllegalArgumentException("Prompt cannot be empty")
        if max_tokens <= 0:
            return list(prompt)
        own = stream is None and use_graph
        stream = Stream.create() if own else stream
        try:
            max_seq = len(prompt) + max_tokens
            cache = self.new_cache(max_seq, stream)
            buffers = self.new_inference_buffers(max_seq)
            self.prefill(prompt, cache, buffers, stream)
            out = self.greedy_decode(cache, buffers, max_tokens - 1, stream, use_graph)
            tokens = list(prompt)
            stops = set(int(s) for s in stop_tokens)
            for t in out:
                if t in stops:
                    break
                tokens.append(int(t))
            return tokens
        finally:
            if own:
                stream.destroy()

    @property
    def weight_bytes(self) -> int:
        """weightBytes (Transformer.kt:395-400): quantized tensors plus fp32 parameters."""
        return sum(w.size_in_bytes for w in self.weights.values()) + sum(b.nbytes for b in self.parameters.values())


class DecodeGraph:
    """A recorded greedy decode step (Transformer.capture_decode): each replay decodes
    one token at the cache's device position and advances it."""

    def __init__(self, handle: ctypes.c_void_p, cache: KVCache, stream: Stream):
        self._h, self.cache, self.stream = handle, cache, stream

    def replay(self, steps: int = 1) -> None:
        self.cache.check_room(steps)
        for _ in range(steps):
            _lib.call("kt_graph_launch", self._h, _stream(self.stream))
            self.cache.length += 1

    def destroy(self) -> None:
        if self._h:
            (self.stream or default_stream()).synchronize()  # no replay still in flight
            _lib.call("kt_graph_destroy", self._h)
            self._h = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass
