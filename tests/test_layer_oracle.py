"""Pins of the prologue / epilogue oracle (oracle/layer.py), CPU only."""

from __future__ import annotations

import numpy as np

from oracle import layer as Lr


def test_sequence_conv_equals_streaming_conv():
    """net/shortconv.py states the two forms are numerically identical."""
    rng = np.random.default_rng(0)
    T, D, K = 23, 7, 4
    x = rng.standard_normal((T, D))
    w = rng.standard_normal((K, D))
    buf0 = rng.standard_normal((K - 1, D))
    seq, new = Lr.short_conv(x, w, buf0)
    buf = buf0.copy()
    for t in range(T):
        y, buf = Lr.short_conv_step(x[t], w, buf)
        np.testing.assert_allclose(y, seq[t], rtol=1e-12, atol=1e-12)
    np.testing.assert_array_equal(buf, new)


def test_conv_equals_numpy_convolve_per_channel():
    rng = np.random.default_rng(1)
    T, D, K = 30, 5, 4
    x = rng.standard_normal((T, D))
    w = rng.standard_normal((K, D))
    out, _ = Lr.short_conv(x, w)
    for c in range(D):
        np.testing.assert_allclose(out[:, c], np.convolve(x[:, c], w[:, c])[:T], rtol=1e-12, atol=1e-12)


def test_prologue_segments_chain_through_the_buffers():
    rng = np.random.default_rng(2)
    B, T, H, d, K = 2, 19, 2, 8, 4
    xs = [rng.standard_normal((B, T, H * d)) for _ in range(3)]
    ws = [rng.standard_normal((K, H * d)) * 0.3 for _ in range(3)]
    q, k, v, bufs = Lr.prologue(*xs, *ws, H)
    q1, k1, v1, b1 = Lr.prologue(*(x[:, :7] for x in xs), *ws, H)
    q2, k2, v2, b2 = Lr.prologue(*(x[:, 7:] for x in xs), *ws, H, bufs=b1)
    np.testing.assert_allclose(np.concatenate([q1, q2], 1), q, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(np.concatenate([v1, v2], 1), v, rtol=1e-12, atol=1e-12)
    for a, b in zip(b2, bufs):
        np.testing.assert_array_equal(a, b)


def test_l2_and_rms_closed_forms():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((5, 16))
    n = np.linalg.norm(Lr.l2_norm(x), axis=-1)
    np.testing.assert_allclose(n, 1.0, rtol=1e-10)
    assert np.all(Lr.l2_norm(np.zeros((2, 16))) == 0.0)
    r = Lr.headwise_rms_norm(x, eps=0.0)
    np.testing.assert_allclose(np.sqrt(np.mean(r * r, axis=-1)), 1.0, rtol=1e-12)
    np.testing.assert_allclose(Lr.swish(np.array([0.0, 1.0])), [0.0, 1.0 / (1.0 + np.exp(-1.0))])
