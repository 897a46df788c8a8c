"""The fused projection + cross-entropy with a quantized head (kt_fused_cross_entropy,
kt_loss.hip) against the oracle's restatement of fusedCrossEntropyLoss
(K/Loss.kt:114-219): the loss, d loss / d hidden and d loss / d bias, with ignored rows,
chunking (the vocabulary's 2^22 / N rows per chunk), accumulate, the reference's argument
errors and repeat calls; ignored rows never change the active rows' results.

Bound: the logits come from the library's products (fp32 combine for up to 16 rows, the
prefill GEMM's fp16 operands above: about 3e-4 normwise per product), so the loss is held
to 2e-3 relative and the gradients to 2e-3 normwise, the path's matmul criterion."""
import numpy as np
import pytest

import oracle
from conftest import normwise_rel
from gpu_helpers import banner, same_bits, upload_quantized

pytestmark = pytest.mark.gpu
IGNORE = -100
TOL = 2e-3


def _setup(kt, oracle_lib, k, n, rows, bits, g, seed, ignore_every=0, std=0.05):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((k, n), dtype=np.float32) * np.float32(std)).astype(np.float32)
    st, q = oracle_lib.quantize(w, bits, g)
    assert st == 0
    del w
    head = kt.QuantizedLinear(k, n, kt.Quantization(bits, g))
    head.weight = upload_quantized(kt, q)
    bias = (rng.standard_normal(n) * 0.1).astype(np.float32)
    head.bias = kt.DeviceTensor.from_numpy(bias.reshape(1, n))
    hidden = rng.standard_normal((rows, k)).astype(np.float32)
    targets = rng.integers(0, n, rows).astype(np.int32)
    if ignore_every:
        targets[1::ignore_every] = IGNORE
    return q, head, bias, hidden, targets


def _run(kt, head, hidden, targets, **kw):
    out = kt.fused_cross_entropy_loss(kt.DeviceTensor.from_numpy(hidden), head, targets, **kw)
    kt.synchronize()
    hg = out.hidden_grad.numpy() if out.hidden_grad is not None else None
    bg = out.bias_grad.numpy().reshape(-1) if out.bias_grad is not None else None
    return out.item(), hg, bg


@pytest.mark.parametrize("k,n,rows,bits,g,ignore_every", [
    (64, 50, 5, 4, 32, 0),          # one-row to small-M products
    (128, 1000, 16, 8, 64, 3),      # row mode
    (896, 4864, 33, 4, 64, 4),      # the prefill GEMM
    (896, 151936, 40, 4, 64, 5),    # Qwen2-0.5B head: 27 rows per chunk, two chunks
    (2048, 32000, 150, 8, 32, 7),   # the 1B head, INT8 g32: 131 rows per chunk
])
def test_matches_the_oracle(kt, oracle_lib, k, n, rows, bits, g, ignore_every):
    banner("fused-ce", k, n, rows, bits, g)
    q, head, bias, hidden, targets = _setup(kt, oracle_lib, k, n, rows, bits, g, k + n, ignore_every)
    loss, hg, bg = _run(kt, head, hidden, targets)
    want_loss, want_hg, want_bg = oracle.fused_cross_entropy(hidden, q, targets, bias, threads=16)
    print(f"  loss {loss:.6f} oracle {want_loss:.6f} hidden {normwise_rel(hg, want_hg):.2e} "
          f"bias {normwise_rel(bg, want_bg):.2e}", flush=True)
    assert abs(loss - want_loss) <= TOL * max(1.0, abs(want_loss))
    assert normwise_rel(hg, want_hg) <= TOL
    assert normwise_rel(bg, want_bg) <= TOL
    assert not hg[targets == IGNORE].any()
    # repeat: the same bits (fixed-order sums, no atomics)
    loss2, hg2, bg2 = _run(kt, head, hidden, targets)
    assert loss2 == loss and same_bits(hg, hg2) and same_bits(bg, bg2)


def test_ignored_rows_do_not_change_the_active_rows(kt, oracle_lib):
    """Chunks are taken over the active rows (Loss.kt:129-133): ignored rows interleaved
    between the same active rows leave the loss and every active row's gradients bit for
    bit as they were, although without compaction the chunks' row counts would change
    (at the Qwen2 head, 27 rows a chunk: 40 active rows are chunks of 27 and 13, the
    prefill GEMM and the small-M kernels), and the ignored rows' gradient is zero."""
    banner("fused-ce-ignored-rows")
    q, head, bias, hidden, targets = _setup(kt, oracle_lib, 896, 151936, 40, 4, 64, 31)
    loss, hg, bg = _run(kt, head, hidden, targets)
    rng = np.random.default_rng(32)
    spread = np.sort(rng.choice(100, 40, replace=False))  # the active rows' places among 100
    hidden2 = rng.standard_normal((100, 896)).astype(np.float32)
    targets2 = np.full(100, IGNORE, np.int32)
    hidden2[spread], targets2[spread] = hidden, targets
    loss2, hg2, bg2 = _run(kt, head, hidden2, targets2)
    assert loss2 == loss and same_bits(hg2[spread], hg) and same_bits(bg2, bg)
    assert not np.delete(hg2, spread, axis=0).any()


def test_accumulate_and_loss_only(kt, oracle_lib):
    banner("fused-ce-accumulate")
    q, head, bias, hidden, targets = _setup(kt, oracle_lib, 256, 700, 20, 4, 64, 11, ignore_every=3)
    loss, hg, bg = _run(kt, head, hidden, targets)
    hg0 = kt.DeviceTensor.from_numpy(np.full(hidden.shape, 0.5, np.float32))
    bg0 = kt.DeviceTensor.from_numpy(np.full((1, 700), -2.0, np.float32))
    out = kt.fused_cross_entropy_loss(kt.DeviceTensor.from_numpy(hidden), head, targets, hidden_grad=hg0,
                                      bias_grad=bg0, accumulate=True)
    kt.synchronize()
    assert out.item() == loss
    np.testing.assert_allclose(out.hidden_grad.numpy(), hg + 0.5, rtol=0, atol=1e-6)
    np.testing.assert_allclose(out.bias_grad.numpy().reshape(-1), bg - 2.0, rtol=0, atol=1e-6)
    loss_only, none_hg, none_bg = _run(kt, head, hidden, targets, grads=False)
    assert loss_only == loss and none_hg is None and none_bg is None


def test_reference_argument_errors_and_empty_loss(kt, oracle_lib):
    banner("fused-ce-errors")
    q, head, bias, hidden, targets = _setup(kt, oracle_lib, 64, 40, 4, 8, 32, 13)
    with pytest.raises(kt.IllegalArgumentException, match="out of bounds"):
        _run(kt, head, hidden, np.array([0, 40, 1, 2]))
    with pytest.raises(kt.IllegalArgumentException, match="out of bounds"):
        _run(kt, head, hidden, np.array([0, -1, 1, 2]))
    with pytest.raises(kt.IllegalArgumentException, match="empty"):
        _run(kt, head, hidden[:0], np.array([], dtype=np.int32))
    # every row ignored: emptyLoss(), no gradient flows (accumulated buffers unchanged)
    hg0 = kt.DeviceTensor.from_numpy(np.full(hidden.shape, 0.25, np.float32))
    bg0 = kt.DeviceTensor.from_numpy(np.full((1, 40), 1.5, np.float32))
    out = kt.fused_cross_entropy_loss(kt.DeviceTensor.from_numpy(hidden), head, [IGNORE] * 4, hidden_grad=hg0,
                                      bias_grad=bg0, accumulate=True)
    kt.synchronize()
    assert out.item() == 0.0
    assert np.all(out.hidden_grad.numpy() == 0.25) and np.all(out.bias_grad.numpy() == 1.5)
