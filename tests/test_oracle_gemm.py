"""Pins the oracle's quantized matmul.

Exact mode is checked against numpy's float64 matmul of the dequantized
weights. Candle mode (int8 activations, integer vec-dots) must equal exact mode
when the activations sit on the int8 grid (quantization is then lossless), and
must stay within the analytic activation-quantization bound otherwise: each
activation moves by at most half a step of its block's scale.
"""
import numpy as np
import pytest

import oracle as O
import synth


def wdeq(t, w, n, k):
    return O.dequantize(t, w, n * k).reshape(n, k).astype(np.float64)


@pytest.mark.parametrize("t", [O.Q8_0, O.Q4_K, O.Q6_K, O.BF16, O.F16])
def test_exact_mode_matches_numpy_f64(t):
    rng = np.random.default_rng(10)
    n, k, m = 64, 512, 9
    _, w, _, _ = synth.weight(rng, t, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    y = O.qmatmul(t, w, n, k, x, O.EXACT)
    want = x.astype(np.float64) @ wdeq(t, w, n, k).T
    assert np.allclose(y, want, rtol=1e-6, atol=1e-6)


def grid_activations(rng, m, k, blk):
    """Rows whose blocks are exactly representable by the activation quantizer."""
    s = np.float32(2.0 ** -5)
    q = rng.integers(-127, 128, (m, k)).astype(np.float32)
    if blk == 32:   # Q8_0: amax = 127 s  ->  d = s
        q[:, ::32] = 127
    else:           # Q8_K: first largest-magnitude element = -128 s  ->  iscale = 1/s
        q[:, ::256] = -128
    return (q * s).astype(np.float32)


@pytest.mark.parametrize("t,blk", [(O.Q8_0, 32), (O.Q4_K, 256), (O.Q6_K, 256)])
def test_candle_mode_equals_exact_on_grid_activations(t, blk):
    rng = np.random.default_rng(11)
    n, k, m = 96, 1024, 5
    _, w, _, _ = synth.weight(rng, t, n, k)
    x = grid_activations(rng, m, k, blk)
    yc = O.qmatmul(t, w, n, k, x, O.CANDLE)
    ye = O.qmatmul(t, w, n, k, x, O.EXACT)
    scale = np.abs(ye).max()
    assert np.max(np.abs(yc - ye)) <= 2e-6 * scale


@pytest.mark.parametrize("t,blk", [(O.Q8_0, 32), (O.Q4_K, 256), (O.Q6_K, 256)])
def test_candle_mode_within_activation_quantization_bound(t, blk):
    rng = np.random.default_rng(12)
    n, k, m = 64, 1024, 6
    _, w, _, _ = synth.weight(rng, t, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    yc = O.qmatmul(t, w, n, k, x, O.CANDLE)
    ye = O.qmatmul(t, w, n, k, x, O.EXACT)
    W = np.abs(wdeq(t, w, n, k))
    xb = np.abs(x).reshape(m, k // blk, blk).max(axis=2)
    step = xb / (127.0 if blk == 32 else 128.0)
    # |sum_k (x_q - x) w| <= sum_blocks step/2 * sum_{k in block} |w|  (+ f16 rounding of d for Q8_0)
    wsum = W.reshape(n, k // blk, blk).sum(axis=2)
    bound = 0.5 * step @ wsum.T
    if blk == 32:
        bound *= 1.0 + 2.0 ** -10 * 127  # the f16 scale's own rounding
    err = np.abs(yc - ye)
    assert np.all(err <= bound * 1.001 + 1e-5)
    # and the bound is not vacuous: the errors are a sizeable fraction of it
    assert err.mean() > 0.01 * bound.mean()


def test_float_weights_are_a_plain_f32_matmul():
    rng = np.random.default_rng(13)
    x = rng.standard_normal((3, 64)).astype(np.float32)
    w = rng.standard_normal((32, 64)).astype(np.float32)
    y = O.qmatmul(O.F32, w.view(np.uint8).reshape(-1), 32, 64, x, O.CANDLE)
    assert np.allclose(y, x @ w.T, rtol=1e-5, atol=1e-5)
