"""The oracle's fused projection + cross-entropy with a quantized head
(kt_oracle_loss.c, restating K/Loss.kt:114-219,236-291), pinned against an
independent fp64 softmax cross-entropy on the dequantized weights, closed forms, the
reference's argument checks and a planted mistake."""
import numpy as np
import pytest

import oracle
from conftest import normwise_rel

IGNORE = -100


def fp64_reference(hidden, q, targets, bias):
    """Textbook softmax cross-entropy in fp64: mean over active rows of logsumexp - l_t,
    and its gradients (softmax - onehot) / active through the dequantized head."""
    w = q.dequantize().astype(np.float64)                       # [K x N]
    h = hidden.astype(np.float64)
    logits = h @ w + (0.0 if bias is None else bias.astype(np.float64))
    t = np.asarray(targets)
    act = np.nonzero(t != IGNORE)[0]
    if act.size == 0:
        return 0.0, np.zeros_like(h), np.zeros(w.shape[1])
    la = logits[act]
    m = la.max(axis=1, keepdims=True)
    lse = m[:, 0] + np.log(np.exp(la - m).sum(axis=1))
    loss = float(np.mean(lse - la[np.arange(act.size), t[act]]))
    p = np.exp(la - lse[:, None])
    p[np.arange(act.size), t[act]] -= 1.0
    g = p / act.size
    hg = np.zeros_like(h)
    hg[act] = g @ w.T
    return loss, hg, g.sum(axis=0)


def _case(seed, k, n, rows, bits, g, ignore_every=0, bias_scale=0.1):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((k, n)) * 0.3).astype(np.float32)
    st, q = oracle.quantize(w, bits, g)
    assert st == 0
    hidden = rng.standard_normal((rows, k)).astype(np.float32)
    targets = rng.integers(0, n, rows)
    if ignore_every:
        targets[::ignore_every] = IGNORE
    bias = (rng.standard_normal(n) * bias_scale).astype(np.float32)
    return hidden, q, targets, bias


@pytest.mark.parametrize("k,n,rows,bits,g,ignore_every", [(64, 50, 5, 4, 32, 0), (96, 333, 17, 8, 32, 3),
                                                         (128, 1000, 9, 4, 64, 2), (40, 7, 4, 8, 16, 0)])
def test_matches_fp64_softmax_cross_entropy(k, n, rows, bits, g, ignore_every):
    hidden, q, targets, bias = _case(k + n, k, n, rows, bits, g, ignore_every)
    loss, hg, bg = oracle.fused_cross_entropy(hidden, q, targets, bias, threads=4)
    want_loss, want_hg, want_bg = fp64_reference(hidden, q, targets, bias)
    assert abs(loss - want_loss) <= 1e-5 * max(1.0, abs(want_loss))
    assert normwise_rel(hg, want_hg) <= 1e-5
    assert normwise_rel(bg, want_bg) <= 1e-5
    # ignored rows receive no gradient
    for r in np.nonzero(np.asarray(targets) == IGNORE)[0]:
        assert not hg[r].any()


def test_chunked_rows_agree():
    """A vocabulary above 2^22 / 8 splits 19 rows into chunks of 8 (Loss.kt:133). The
    reference sums a row's 2^19 exponentials one after another in fp32: that sum's own
    rounding (up to n ulps; 3e-4 relative measured here) bounds the loss and, through
    1 / sum, every probability, so the loss is held to 2e-3 absolute and the gradients to
    1e-3 normwise."""
    hidden, q, targets, bias = _case(5, 32, (1 << 19) + 3, 19, 4, 32, ignore_every=5, bias_scale=1.0)
    loss, hg, bg = oracle.fused_cross_entropy(hidden, q, targets, bias, threads=8)
    want_loss, want_hg, want_bg = fp64_reference(hidden, q, targets, bias)
    assert abs(loss - want_loss) <= 2e-3
    assert normwise_rel(hg, want_hg) <= 1e-3
    assert normwise_rel(bg, want_bg) <= 1e-3


def test_closed_forms():
    k, n = 32, 40
    zero_w = np.zeros((k, n), dtype=np.float32)
    st, q = oracle.quantize(zero_w, 8, 32)
    hidden = np.random.default_rng(1).standard_normal((6, k)).astype(np.float32)
    targets = np.array([0, 3, IGNORE, 39, 3, 7])
    # uniform logits: loss = ln N, bias gradient (1/N - [v == t]) / active summed, no hidden gradient
    loss, hg, bg = oracle.fused_cross_entropy(hidden, q, targets, None)
    assert abs(loss - np.log(n)) <= 1e-6 * np.log(n)
    act = targets[targets != IGNORE]
    want_bg = np.full(n, act.size / n) - np.bincount(act, minlength=n)
    np.testing.assert_allclose(bg, want_bg / act.size, rtol=0, atol=1e-7)
    assert not hg.any()
    # one dominant logit: at the target the loss vanishes, elsewhere it is the gap
    bias = np.zeros(n, dtype=np.float32)
    bias[3] = 60.0
    loss, _, _ = oracle.fused_cross_entropy(hidden[:1], q, [3], bias)
    assert loss < 1e-20
    loss, _, _ = oracle.fused_cross_entropy(hidden[:1], q, [4], bias)
    assert abs(loss - 60.0) <= 1e-5


def test_reference_argument_checks():
    hidden, q, targets, bias = _case(2, 16, 10, 3, 4, 16)
    loss, hg, bg = oracle.fused_cross_entropy(hidden, q, [IGNORE] * 3, bias)
    assert loss == 0.0 and not hg.any() and not bg.any()    # emptyLoss()
    with pytest.raises(ValueError):
        oracle.fused_cross_entropy(hidden, q, [0, 10, 1], bias)   # target out of bounds
    with pytest.raises(ValueError):
        oracle.fused_cross_entropy(hidden, q, [0, -1, 1], bias)   # negative, not ignore_index
    with pytest.raises(ValueError):
        oracle.fused_cross_entropy(hidden[:0], q, [], bias)       # targets cannot be empty


def test_planted_mistake_is_caught():
    """The checks above would catch a plausible slip: averaging over all rows instead of
    the active ones (ignored rows counted) moves the loss and gradients off the fp64
    reference by the ignored fraction."""
    hidden, q, targets, bias = _case(3, 64, 77, 9, 4, 32, ignore_every=3)
    loss, hg, bg = oracle.fused_cross_entropy(hidden, q, targets, bias)
    active = int(np.sum(np.asarray(targets) != IGNORE))
    slip = active / len(targets)
    want_loss, want_hg, _ = fp64_reference(hidden, q, targets, bias)
    assert abs(loss * slip - want_loss) > 1e-3 * abs(want_loss)
    assert normwise_rel(hg * slip, want_hg) > 1e-3
