"""Pins the oracle's decoder pieces (oracle/kt_oracle_decoder.c) and its decoder
orchestration (oracle/decoder_ref.py) without a GPU.

Each piece is checked against what the mathematics fixes -- closed forms in fp64,
identities (position 0, a single cached position, equal scores), invariants (pair norms
under rotation, composition of rotations, per-head independence from
RegressionTest.kt:57-76) -- and the orchestration against the reference's own
consistency tests (PrefillTest.kt:36-138): prefill across chunk boundaries equals
one-token decoding, a prefill continued from an existing cache equals one long prefill,
and generate equals argmax over teacher-forced decoding.
"""
import math

import numpy as np
import pytest

import oracle
from conftest import normwise_rel as normwise
from oracle import decoder_ref


def ulp_close(a, b, ulps=2):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    tol = ulps * np.spacing(np.maximum(np.abs(a), np.abs(b)).astype(np.float32))
    return bool(np.all(np.abs(a.astype(np.float64) - b.astype(np.float64)) <= tol))


# ---- RoPE frequencies ---------------------------------------------------------------

def test_inv_freq_closed_form():
    for hd, base in [(64, 500000.0), (128, 10000.0), (8, 10000.0)]:
        got = oracle.rope_inv_freq(hd, base)
        want = np.array([1.0 / base ** ((2 * i) / hd) for i in range(hd // 2)])
        assert ulp_close(got, want.astype(np.float32), 2), (hd, base)
    assert oracle.rope_inv_freq(8, 10000.0).tolist() == [1.0, np.float32(0.1), np.float32(0.01), np.float32(0.001)]


def test_inv_freq_scaling_regimes():
    """RoPEScaling.scale: short wavelengths unchanged, long ones divided by the factor,
    the band between blended (Llama 3.1's factor 8, 1, 4, 8192)."""
    hd, base, scaling = 128, 500000.0, (8.0, 1.0, 4.0, 8192)
    raw = oracle.rope_inv_freq(hd, base)
    got = oracle.rope_inv_freq(hd, base, scaling)
    blended = 0
    for r, g in zip(raw, got):
        wavelength = 2 * math.pi / float(r)
        if wavelength < 8192 / 4:
            assert g == r
        elif wavelength > 8192 / 1:
            assert ulp_close(g, np.float32(r / np.float32(8.0)), 1)
        else:
            smooth = (8192 / wavelength - 1.0) / (4.0 - 1.0)
            want = (1 - smooth) * float(r) / 8.0 + smooth * float(r)
            assert abs(float(g) - want) <= 4e-7 * abs(want)
            assert float(r) / 8.0 <= float(g) * (1 + 1e-6) and float(g) <= float(r) * (1 + 1e-6)
            blended += 1
    assert blended > 0


# ---- RMSNorm ------------------------------------------------------------------------

def test_rmsnorm_closed_form_and_special_rows():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((5, 96)).astype(np.float32)
    w = rng.standard_normal(96).astype(np.float32)
    eps = 1e-5
    got = oracle.rmsnorm(x, w, eps)
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + eps) * w
    np.testing.assert_allclose(got, want, rtol=2e-6, atol=1e-7)
    zero = oracle.rmsnorm(np.zeros((1, 8), np.float32), np.ones(8, np.float32), eps)
    assert np.all(zero == 0)
    const = oracle.rmsnorm(np.full((1, 16), 3.0, np.float32), np.ones(16, np.float32), 1e-6)
    assert ulp_close(const, np.full(16, 3.0 / math.sqrt(9.0 + 1e-6), np.float32), 2)
    # scaling the row by a power of two leaves the result unchanged when eps is negligible
    np.testing.assert_allclose(oracle.rmsnorm(x * 4, w, 0.0), oracle.rmsnorm(x, w, 0.0), rtol=1e-6)


# ---- RoPE rotation ------------------------------------------------------------------

def test_rope_identities_and_closed_form():
    rng = np.random.default_rng(2)
    hd, heads, tokens = 16, 3, 6
    inv = oracle.rope_inv_freq(hd, 10000.0)
    rows = rng.standard_normal((tokens, heads * hd)).astype(np.float32)
    # position 0 is the identity (cos 0 = 1, sin 0 = 0 exactly)
    assert np.array_equal(oracle.rope_rows(rows[:1], hd, inv, 0), rows[:1])
    out = oracle.rope_rows(rows, hd, inv, 5)
    half = hd // 2
    for t in range(tokens):
        for h in range(heads):
            a = rows[t, h * hd:(h + 1) * hd].astype(np.float64)
            b = out[t, h * hd:(h + 1) * hd].astype(np.float64)
            theta = (5 + t) * inv.astype(np.float64)
            want1 = a[:half] * np.cos(theta) - a[half:] * np.sin(theta)
            want2 = a[:half] * np.sin(theta) + a[half:] * np.cos(theta)
            np.testing.assert_allclose(b, np.concatenate([want1, want2]), rtol=0, atol=3e-6 * (1 + 5 + t))
            # pair norms are kept
            np.testing.assert_allclose(np.hypot(b[:half], b[half:]), np.hypot(a[:half], a[half:]), rtol=2e-6)
    # rotating by 3 then by 4 equals rotating by 7
    two = oracle.rope_rows(oracle.rope_rows(rows[:1], hd, inv, 3), hd, inv, 4)
    np.testing.assert_allclose(two, oracle.rope_rows(rows[:1], hd, inv, 7), atol=2e-6)
    # every head rotates alike (RegressionTest.kt:57-76) and rows agree with one row at a time
    for h in range(heads):
        one = oracle.rope_rows(np.ascontiguousarray(rows[:, h * hd:(h + 1) * hd]), hd, inv, 5)
        np.testing.assert_array_equal(one, out[:, h * hd:(h + 1) * hd])
    for t in range(tokens):
        np.testing.assert_array_equal(oracle.rope_rows(rows[t:t + 1], hd, inv, 5 + t), out[t:t + 1])


# ---- attention ----------------------------------------------------------------------

def _cache(rng, layers, kvh, max_seq, hd, length):
    keys = np.zeros(layers * kvh * max_seq * hd, np.float32)
    values = np.zeros_like(keys)
    view_k = keys.reshape(layers, kvh, max_seq, hd)
    view_v = values.reshape(layers, kvh, max_seq, hd)
    view_k[:, :, :length] = rng.standard_normal((layers, kvh, length, hd))
    view_v[:, :, :length] = rng.standard_normal((layers, kvh, length, hd))
    return keys, values


def test_attention_brute_force_causal_gqa():
    rng = np.random.default_rng(3)
    layers, heads, kvh, hd, max_seq = 2, 8, 2, 16, 40
    start, tokens = 20, 7
    keys, values = _cache(rng, layers, kvh, max_seq, hd, start + tokens)
    q = rng.standard_normal((tokens, heads * hd)).astype(np.float32)
    for layer in range(layers):
        got = oracle.attend(q, start, keys, values, layer, heads, kvh, hd, max_seq)
        K = keys.reshape(layers, kvh, max_seq, hd)[layer].astype(np.float64)
        V = values.reshape(layers, kvh, max_seq, hd)[layer].astype(np.float64)
        for t in range(tokens):
            pos = start + t
            for h in range(heads):
                g = h // (heads // kvh)
                s = K[g, :pos + 1] @ q[t, h * hd:(h + 1) * hd].astype(np.float64) / math.sqrt(hd)
                p = np.exp(s - s.max())
                p /= p.sum()
                want = p @ V[g, :pos + 1]
                np.testing.assert_allclose(got[t, h * hd:(h + 1) * hd], want, rtol=0, atol=2e-6)


def test_attention_identities():
    rng = np.random.default_rng(4)
    hd, max_seq = 8, 6
    keys, values = _cache(rng, 1, 1, max_seq, hd, 6)
    q = rng.standard_normal((1, hd)).astype(np.float32)
    # position 0: the single cached value, exactly
    got = oracle.attend(q, 0, keys, values, 0, 1, 1, hd, max_seq)
    np.testing.assert_array_equal(got[0], values[:hd])
    # equal keys: the mean of the values
    k2 = keys.copy().reshape(max_seq, hd)
    k2[:] = k2[0]
    got = oracle.attend(q, 5, k2.reshape(-1), values, 0, 1, 1, hd, max_seq)
    np.testing.assert_allclose(got[0], values.reshape(max_seq, hd).mean(axis=0), atol=1e-6)


# ---- SwiGLU gate and argmax ---------------------------------------------------------

def test_silu_mul_closed_form():
    rng = np.random.default_rng(5)
    g = (rng.standard_normal(1000) * 4).astype(np.float32)
    u = rng.standard_normal(1000).astype(np.float32)
    got = oracle.silu_mul(g, u)
    g64 = g.astype(np.float64)
    np.testing.assert_allclose(got, g64 / (1 + np.exp(-g64)) * u, rtol=3e-7, atol=1e-30)
    assert oracle.silu_mul(np.zeros(3, np.float32), np.ones(3, np.float32)).tolist() == [0.0, 0.0, 0.0]


def test_argmax_rules():
    assert oracle.argmax(np.array([1, 5, 5, 2], np.float32)) == 1          # first maximum
    assert oracle.argmax(np.array([-2e9, -3e9], np.float32)) == 0           # nothing above -1e9
    assert oracle.argmax(np.array([np.nan, 1.0, np.nan, 3.0], np.float32)) == 3  # NaN never wins
    assert oracle.argmax(np.array([-1e9, -5e8], np.float32)) == 1           # strictly above the floor
    rng = np.random.default_rng(6)
    x = rng.standard_normal(32000).astype(np.float32)
    assert oracle.argmax(x) == int(np.argmax(x))


# ---- the orchestration --------------------------------------------------------------

def small_model(bits=4, tied=False, seed=7, cfg=None):
    cfg = cfg or decoder_ref.Config(vocabulary_size=61, dimension=64, num_layers=2, num_heads=4,
                                    hidden_dimension=96, num_key_value_heads=2, norm_eps=1e-6, rope_theta=10000.0)
    rng = np.random.default_rng(seed)
    shapes = {"lmHead": (cfg.dimension, cfg.vocabulary_size)}
    if not tied:
        shapes["embedding"] = (cfg.vocabulary_size, cfg.dimension)
    for l in range(cfg.num_layers):
        p = f"block.{l}."
        shapes[p + "attention.wQ"] = (cfg.dimension, cfg.dimension)
        shapes[p + "attention.wK"] = (cfg.dimension, cfg.kv_dimension)
        shapes[p + "attention.wV"] = (cfg.dimension, cfg.kv_dimension)
        shapes[p + "attention.wOut"] = (cfg.dimension, cfg.dimension)
        shapes[p + "ffn.wGate"] = (cfg.dimension, cfg.hidden_dimension)
        shapes[p + "ffn.wUp"] = (cfg.dimension, cfg.hidden_dimension)
        shapes[p + "ffn.wDown"] = (cfg.hidden_dimension, cfg.dimension)
    quantized, fp32 = {}, {}
    for name, (k, n) in shapes.items():
        w = (rng.standard_normal((k, n)) * 0.3).astype(np.float32)
        status, q = oracle.quantize(w, bits, 32)
        assert status == 0
        quantized[name], fp32[name] = q, w
    norms = {f"block.{l}.norm{i}": (1 + 0.1 * rng.standard_normal(cfg.dimension)).astype(np.float32)
             for l in range(cfg.num_layers) for i in (1, 2)}
    norms["finalNorm"] = (1 + 0.1 * rng.standard_normal(cfg.dimension)).astype(np.float32)
    return decoder_ref.RefTransformer(cfg, quantized, norms, tied=tied), fp32


@pytest.mark.parametrize("bits,tied", [(4, False), (8, False), (4, True)])
def test_prefill_across_chunks_equals_token_by_token(bits, tied):
    model, _ = small_model(bits, tied)
    rng = np.random.default_rng(8)
    for length in (1, 31, 32, 33, 70):
        prompt = rng.integers(0, model.config.vocabulary_size, length).tolist()
        c1 = model.new_cache(length + 1)
        logits = model.prefill(prompt, c1)
        c2 = model.new_cache(length + 1)
        for t in prompt:
            last = model.decode(t, c2)
        assert c1.length == c2.length == length
        assert np.max(np.abs(logits - last)) <= 1e-4
        assert np.max(np.abs(c1.keys - c2.keys)) <= 1e-4
        assert np.max(np.abs(c1.values - c2.values)) <= 1e-4


def test_continued_prefill_and_generate():
    model, _ = small_model()
    rng = np.random.default_rng(9)
    prompt = rng.integers(0, model.config.vocabulary_size, 50).tolist()
    whole = model.prefill(prompt, model.new_cache(50))
    cache = model.new_cache(50)
    model.prefill(prompt[:20], cache)
    assert np.max(np.abs(model.prefill(prompt[20:], cache) - whole)) <= 1e-4
    generated = model.generate(prompt[:45], 12)
    cache = model.new_cache(57)
    logits = model.prefill(prompt[:45], cache)
    expected = []
    for step in range(12):
        best = int(np.argmax(logits))
        expected.append(best)
        if step < 11:
            logits = model.decode(best, cache)
    assert generated == prompt[:45] + expected


def test_decoder_against_an_fp64_forward():
    """One fp64 forward pass of the dequantized model (every operation in float64)
    agrees with prefill: the orchestration wires the pieces as the reference does."""
    model, _ = small_model(4)
    c = model.config
    prompt = [3, 17, 8, 29, 40, 2]
    logits = model.prefill(prompt, model.new_cache(len(prompt)))
    deq = {k: v.dequantize().astype(np.float64) for k, v in model.quantized.items()}
    x = np.stack([deq["embedding"][t] for t in prompt])
    T, hd = len(prompt), c.head_dim
    inv = oracle.rope_inv_freq(hd, c.rope_theta).astype(np.float64)

    def norm(v, w):
        return v / np.sqrt((v ** 2).mean(axis=1, keepdims=True) + c.norm_eps) * w

    def rope(m):
        out = m.copy()
        for t in range(T):
            th = t * inv
            for h in range(m.shape[1] // hd):
                a, b = m[t, h * hd:h * hd + hd // 2], m[t, h * hd + hd // 2:(h + 1) * hd]
                out[t, h * hd:h * hd + hd // 2] = a * np.cos(th) - b * np.sin(th)
                out[t, h * hd + hd // 2:(h + 1) * hd] = a * np.sin(th) + b * np.cos(th)
        return out

    for l in range(c.num_layers):
        p = f"block.{l}."
        n1 = norm(x, model.norms[p + "norm1"])
        q, k, v = rope(n1 @ deq[p + "attention.wQ"]), rope(n1 @ deq[p + "attention.wK"]), n1 @ deq[p + "attention.wV"]
        ctx = np.zeros_like(q)
        g = c.num_heads // c.num_key_value_heads
        for h in range(c.num_heads):
            kh = k[:, (h // g) * hd:(h // g + 1) * hd]
            vh = v[:, (h // g) * hd:(h // g + 1) * hd]
            s = q[:, h * hd:(h + 1) * hd] @ kh.T / math.sqrt(hd)
            s[np.triu_indices(T, 1)] = -np.inf
            pr = np.exp(s - s.max(axis=1, keepdims=True))
            pr /= pr.sum(axis=1, keepdims=True)
            ctx[:, h * hd:(h + 1) * hd] = pr @ vh
        x = x + ctx @ deq[p + "attention.wOut"]
        n2 = norm(x, model.norms[p + "norm2"])
        gate = n2 @ deq[p + "ffn.wGate"]
        x = x + (gate / (1 + np.exp(-gate)) * (n2 @ deq[p + "ffn.wUp"])) @ deq[p + "ffn.wDown"]
    want = norm(x[-1:], model.norms["finalNorm"]) @ deq["lmHead"]
    np.testing.assert_allclose(logits, want[0], rtol=0, atol=2e-4 * np.abs(want).max())


def test_dense_mode_agrees_with_the_restated_loops():
    """RefTransformer(dense=True) -- BLAS products over the fully dequantized weights and
    float64 attention -- gives the restated loops' prefill, cache and decode logits up to
    summation order (normwise 1e-5), and attend_dense agrees with oracle.attend (causal,
    GQA, a prefix already in the cache)."""
    model, _ = small_model(4)
    dense = decoder_ref.RefTransformer(model.config, model.quantized, model.norms, dense=True)
    rng = np.random.default_rng(31)
    prompt = rng.integers(0, model.config.vocabulary_size, 45).tolist()
    c1, c2 = model.new_cache(49), dense.new_cache(49)
    a, b = model.prefill(prompt, c1), dense.prefill(prompt, c2)
    assert normwise(b, a) <= 1e-5 and normwise(c2.keys, c1.keys) <= 1e-5 and normwise(c2.values, c1.values) <= 1e-5
    for t in rng.integers(0, model.config.vocabulary_size, 4).tolist():
        assert normwise(dense.decode(t, c2), model.decode(t, c1)) <= 1e-5
    heads, kvh, hd, ms, layers = 8, 2, 16, 40, 2
    keys = rng.standard_normal(layers * kvh * ms * hd).astype(np.float32)
    values = rng.standard_normal(layers * kvh * ms * hd).astype(np.float32)
    for start, tokens in ((0, 7), (13, 5), (30, 1)):
        q = rng.standard_normal((tokens, heads * hd)).astype(np.float32)
        want = oracle.attend(q, start, keys, values, 1, heads, kvh, hd, ms)
        got = decoder_ref.attend_dense(q, start, keys, values, 1, heads, kvh, hd, ms)
        np.testing.assert_allclose(got, want, rtol=0, atol=2e-6)


def test_vectorised_dequantize_equals_the_row_accessor():
    """oracle.Quantized.dequantize (numpy) is dequantize_row (C) bit for bit, INT8 with and
    without a partial last group, INT4 with an odd column count."""
    rng = np.random.default_rng(32)
    for k, n, bits, g in ((100, 37, 4, 32), (70, 9, 4, 64), (65, 130, 8, 64), (33, 40, 8, 16)):
        status, q = oracle.quantize((rng.standard_normal((k, n)) * 0.3).astype(np.float32), bits, g)
        assert status == 0
        full = q.dequantize()
        for r in range(k):
            assert np.array_equal(full[r].view(np.uint32), q.dequantize_row(r).view(np.uint32))
