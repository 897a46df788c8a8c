"""The oracle for the quantized decoder: Transformer.prefill / decode / generate over
the oracle's quantized matmul and decoder pieces.

TEST INFRASTRUCTURE ONLY (the checker of kotensor_amd.transformer); the product never
imports it. Reference citations are relative to Engine/kotensor/src/main/kotlin/.

  RefTransformer.prefill -- Transformer.prefill / prefillLayers (Transformer.kt:99-132):
                            chunks of MatMul.TILE_M = 32 rows (MatMul.kt:16), every layer
                            per chunk (TransformerBlock.prefillInto, :213-220;
                            Attention.prefillInto, Attention.kt:241-275), then the final
                            norm and lmHead on the last row.
  RefTransformer.decode  -- Transformer.decode (Transformer.kt:141-154) with
                            TransformerBlock.decodeInto (:204-211) and
                            Attention.decodeInto (Attention.kt:207-239).
  RefTransformer.generate -- greedy streamFrom (Transformer.kt:211-233) with
                            argmaxOfLastToken.

The quantized embedding row is QuantizedTensor.dequantizeRow (QuantizedEmbedding,
Embedding.kt:96-101); a tied model reads head columns (TiedQuantizedEmbedding,
Embedding.kt:130-135). Pinning: the pieces are pinned in tests/test_oracle_decoder.py;
the orchestration is checked there against the reference's own consistency properties
(prefill across chunk boundaries equals one-token decoding; a continued prefill equals
one long prefill; generate equals argmax of teacher-forced decoding).

dense=True replaces the two costly pieces with brute force for models whose restated
loops would take minutes (the 1B decoder over a 1024-token prompt): every projection is
x . W with W the fully dequantized fp32 weight (value(r, c) of every element, the same
numbers the reference's kernels multiply) through numpy's BLAS, and the cached attention
is the same softmax over the same keys in float64. Each differs from the restated loops
by summation order only; tests/test_oracle_decoder.py bounds the difference.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

import oracle

TILE_M = 32  # MatMul.TILE_M (MatMul.kt:16): the prefill chunk


def attend_dense(q: np.ndarray, start: int, keys: np.ndarray, values: np.ndarray, layer: int, num_heads: int,
                 num_kv_heads: int, head_dim: int, max_seq: int) -> np.ndarray:
    """attendCached (Attention.kt:277-349) as oracle.attend computes it -- token t at
    position start + t attends to cached positions 0..start + t of the kv head of its
    query head, softmax of q . k / sqrt(head_dim), times v -- in float64 matrix form."""
    tokens = q.shape[0]
    group = num_heads // num_kv_heads
    kv = keys.reshape(-1, num_kv_heads, max_seq, head_dim)[layer, :, :start + tokens].astype(np.float64)
    vv = values.reshape(-1, num_kv_heads, max_seq, head_dim)[layer, :, :start + tokens].astype(np.float64)
    qh = q.reshape(tokens, num_heads, head_dim).astype(np.float64)
    scale = np.float64(np.float32(1.0) / np.float32(np.sqrt(np.float64(np.float32(head_dim)))))
    visible = np.arange(start + tokens)[None, :] <= (start + np.arange(tokens))[:, None]
    out = np.empty((tokens, num_heads, head_dim), dtype=np.float64)
    for h in range(num_heads):
        s = (qh[:, h] @ kv[h // group].T) * scale
        s = np.where(visible, s, -np.inf)
        p = np.exp(s - s.max(axis=1, keepdims=True))
        out[:, h] = (p / p.sum(axis=1, keepdims=True)) @ vv[h // group]
    return out.reshape(tokens, num_heads * head_dim).astype(np.float32)


@dataclass
class Config:
    vocabulary_size: int
    dimension: int
    num_layers: int
    num_heads: int
    hidden_dimension: int
    num_key_value_heads: int
    norm_eps: float = 1e-6
    rope_theta: float = 10000.0
    rope_scaling: tuple | None = None  # (factor, low, high, original_max)

    @property
    def head_dim(self) -> int:
        return self.dimension // self.num_heads

    @property
    def kv_dimension(self) -> int:
        return self.num_key_value_heads * self.head_dim


@dataclass
class RefCache:
    """KVCache (KVCache.kt:3-59): keys/values [layers x kv_heads x max_seq x head_dim]."""
    keys: np.ndarray
    values: np.ndarray
    max_sequence_length: int
    length: int = 0


@dataclass
class RefTransformer:
    config: Config
    quantized: dict  # name -> oracle.Quantized ("embedding" unless tied, blocks, "lmHead")
    norms: dict      # name -> fp32 [dimension] ("block.l.norm1", "block.l.norm2", "finalNorm")
    tied: bool = False
    biases: dict = field(default_factory=dict)  # name -> fp32 [out]; QuantizedLinear.bias (QuantizedLinear.kt:16-25)
    dense: bool = False  # brute-force projections and attention (see the module docstring)
    inv_freq: np.ndarray = field(init=False)
    _dense_weights: dict = field(init=False, default_factory=dict)

    def __post_init__(self):
        c = self.config
        self.inv_freq = oracle.rope_inv_freq(c.head_dim, c.rope_theta, c.rope_scaling)

    def new_cache(self, max_sequence_length: int) -> RefCache:
        c = self.config
        n = c.num_layers * c.num_key_value_heads * max_sequence_length * c.head_dim
        return RefCache(np.zeros(n, np.float32), np.zeros(n, np.float32), max_sequence_length)

    # -- pieces ----------------------------------------------------------------------
    def _project(self, x: np.ndarray, name: str) -> np.ndarray:
        """QuantizedLinear.forwardInto: the product, then += bias."""
        if self.dense:
            w = self._dense_weights.get(name)
            if w is None:
                w = self._dense_weights[name] = self.quantized[name].dequantize()
            out = np.matmul(x.astype(np.float32), w)
        else:
            out = oracle.multiply_quantized(x, self.quantized[name], x.shape[0], threads=16)
        if name in self.biases:
            out = (out + self.biases[name][None, :]).astype(np.float32)
        return out

    def embed(self, tokens) -> np.ndarray:
        if self.tied:
            w = self.quantized["lmHead"]
            return np.stack([w.dequantize_column(int(t)) for t in tokens]).astype(np.float32)
        w = self.quantized["embedding"]
        return np.stack([w.dequantize_row(int(t)) for t in tokens]).astype(np.float32)

    def _layer(self, x: np.ndarray, cache: RefCache, layer: int) -> np.ndarray:
        """TransformerBlock.prefillInto / decodeInto on rows x at cache.length + t."""
        c = self.config
        p = f"block.{layer}."
        start = cache.length
        normed = oracle.rmsnorm(x, self.norms[p + "norm1"], c.norm_eps)
        q = self._project(normed, p + "attention.wQ")
        k = self._project(normed, p + "attention.wK")
        v = self._project(normed, p + "attention.wV")
        q = oracle.rope_rows(q, c.head_dim, self.inv_freq, start)
        k = oracle.rope_rows(k, c.head_dim, self.inv_freq, start)
        tokens = x.shape[0]
        hd, kvh, ms = c.head_dim, c.num_key_value_heads, cache.max_sequence_length
        for h in range(kvh):
            for t in range(tokens):
                off = ((layer * kvh + h) * ms + start + t) * hd
                cache.keys[off:off + hd] = k[t, h * hd:(h + 1) * hd]
                cache.values[off:off + hd] = v[t, h * hd:(h + 1) * hd]
        if self.dense:
            context = attend_dense(q, start, cache.keys, cache.values, layer, c.num_heads, kvh, hd, ms)
        else:
            context = oracle.attend(q, start, cache.keys, cache.values, layer, c.num_heads, kvh, hd, ms)
        x = (x + self._project(context, p + "attention.wOut")).astype(np.float32)
        normed = oracle.rmsnorm(x, self.norms[p + "norm2"], c.norm_eps)
        gate = self._project(normed, p + "ffn.wGate")
        up = self._project(normed, p + "ffn.wUp")
        fused = oracle.silu_mul(gate, up)
        return (x + self._project(fused, p + "ffn.wDown")).astype(np.float32)

    def _head(self, last_row: np.ndarray) -> np.ndarray:
        normed = oracle.rmsnorm(last_row.reshape(1, -1), self.norms["finalNorm"], self.config.norm_eps)
        return self._project(normed, "lmHead")[0]

    # -- the reference's entry points -------------------------------------------------
    def prefill(self, prompt, cache: RefCache) -> np.ndarray:
        if len(prompt) == 0:
            raise ValueError("Prompt cannot be empty")
        if cache.length + len(prompt) > cache.max_sequence_length:
            raise ValueError("KV cache full")
        x = None
        for start in range(0, len(prompt), TILE_M):
            chunk = prompt[start:start + TILE_M]
            x = self.embed(chunk)
            for layer in range(self.config.num_layers):
                x = self._layer(x, cache, layer)
            cache.length += len(chunk)
        return self._head(x[-1])

    def decode(self, token: int, cache: RefCache) -> np.ndarray:
        if cache.length + 1 > cache.max_sequence_length:
            raise ValueError("KV cache full")
        x = self.embed([token])
        for layer in range(self.config.num_layers):
            x = self._layer(x, cache, layer)
        cache.length += 1
        return self._head(x[0])

    def generate(self, prompt, max_tokens: int) -> list[int]:
        cache = self.new_cache(len(prompt) + max_tokens)
        logits = self.prefill(prompt, cache)
        out = list(prompt)
        for step in range(max_tokens):
            nxt = oracle.argmax(logits)
            out.append(nxt)
            if step < max_tokens - 1:
                logits = self.decode(nxt, cache)
        return out
