"""Pins of the prologue / epilogue oracle (oracle/layer.py), CPU only."""

from __future__ import annotations

import numpy as np
import pytest

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


def _fd(f, x, direction, h=1e-6):
    return (f(x + h * direction) - f(x - h * direction)) / (2 * h)


def test_prologue_bwd_matches_finite_differences():
    """<dL, dx> == directional derivative of L = <dy, prologue(x)> for every input."""
    rng = np.random.default_rng(11)
    B, T, H, d, K = 2, 9, 2, 6, 4
    xs = [rng.standard_normal((B, T, H * d)) for _ in range(3)]
    ws = [rng.standard_normal((K, H * d)) * 0.4 for _ in range(3)]
    bufs = [rng.standard_normal((B, K - 1, H * d)) for _ in range(3)]
    dys = [rng.standard_normal((B, T, H, d)) for _ in range(3)]

    def loss(xs_, ws_, bufs_):
        q, k, v, _ = Lr.prologue(*xs_, *ws_, H, bufs=bufs_)
        return sum(np.sum(a * b) for a, b in zip((q, k, v), dys))

    dx0, dx1, dx2, dws, dbs = Lr.prologue_bwd(*xs, *ws, H, *dys, bufs=bufs)
    dxs = [dx0, dx1, dx2]
    for n in range(3):
        u = rng.standard_normal(xs[n].shape)
        xs_p = [x.copy() for x in xs]
        fd = (loss([x + 1e-6 * u if i == n else x for i, x in enumerate(xs)], ws, bufs)
              - loss([x - 1e-6 * u if i == n else x for i, x in enumerate(xs)], ws, bufs)) / 2e-6
        np.testing.assert_allclose(np.sum(dxs[n] * u), fd, rtol=1e-6, atol=1e-8)
        u = rng.standard_normal(ws[n].shape)
        fd = (loss(xs, [w + 1e-6 * u if i == n else w for i, w in enumerate(ws)], bufs)
              - loss(xs, [w - 1e-6 * u if i == n else w for i, w in enumerate(ws)], bufs)) / 2e-6
        np.testing.assert_allclose(np.sum(dws[n] * u), fd, rtol=1e-6, atol=1e-8)
        u = rng.standard_normal(bufs[n].shape)
        fd = (loss(xs, ws, [b + 1e-6 * u if i == n else b for i, b in enumerate(bufs)])
              - loss(xs, ws, [b - 1e-6 * u if i == n else b for i, b in enumerate(bufs)])) / 2e-6
        np.testing.assert_allclose(np.sum(dbs[n] * u), fd, rtol=1e-6, atol=1e-8)


def test_epilogue_bwd_matches_finite_differences():
    rng = np.random.default_rng(12)
    B, T, H, dv = 2, 5, 3, 8
    o = rng.standard_normal((B, T, H, dv))
    z = rng.standard_normal((B, T, H * dv))
    dy = rng.standard_normal((B, T, H * dv))
    do, dz = Lr.epilogue_bwd(o, z, dy)
    u = rng.standard_normal(o.shape)
    fd = (np.sum(dy * Lr.epilogue(o + 1e-6 * u, z)) - np.sum(dy * Lr.epilogue(o - 1e-6 * u, z))) / 2e-6
    np.testing.assert_allclose(np.sum(do * u), fd, rtol=1e-6, atol=1e-9)
    u = rng.standard_normal(z.shape)
    fd = (np.sum(dy * Lr.epilogue(o, z + 1e-6 * u)) - np.sum(dy * Lr.epilogue(o, z - 1e-6 * u))) / 2e-6
    np.testing.assert_allclose(np.sum(dz * u), fd, rtol=1e-6, atol=1e-9)


def test_l2_norm_gradient_at_a_zero_row_is_zero():
    """net/tests/test_22_l2norm_padding_gradient.py: zero rows give exactly zero gradient and do
    not change the other rows' gradients."""
    x = np.array([[3.0, 4.0, 0.0, 0.0], [0.0, 0.0, 0.0, 0.0], [1.0, 0.0, 0.0, 0.0]])
    dy = np.ones_like(x)
    g = Lr.l2_norm_bwd(x, dy)
    assert np.all(np.isfinite(g)) and np.all(g[1] == 0.0)
    np.testing.assert_allclose(g[[0, 2]], Lr.l2_norm_bwd(x[[0, 2]], dy[[0, 2]]), rtol=0, atol=0)
    # and the nonzero rows equal the finite-difference gradient of the plain expression
    u = np.random.default_rng(13).standard_normal((2, 4))
    fd = (np.sum(Lr.l2_norm(x[[0, 2]] + 1e-6 * u)) - np.sum(Lr.l2_norm(x[[0, 2]] - 1e-6 * u))) / 2e-6
    np.testing.assert_allclose(np.sum(g[[0, 2]] * u), fd, rtol=1e-6)


# ---------------------------------------------------------------------------
# composition order of the prologue and epilogue (net/kda.py:194-214)
# ---------------------------------------------------------------------------


def _indep_swish_conv(x, w):
    """swish(causal depthwise conv) of one sequence (T, D) by numpy.convolve and
    scipy's logistic function, independent of the oracle's own routines."""
    from scipy.special import expit
    T, D = x.shape
    a = np.stack([np.convolve(x[:, c], w[:, c])[:T] for c in range(D)], axis=1)
    return a * expit(a)


def test_prologue_order_conv_swish_then_l2_on_q_k_only():
    """q and k are swish(conv(x)) / (||.|| + 1e-12) per head row; v is swish(conv(x))
    with no norm.  Catches: L2 before swish (rows not unit norm), v normalised,
    the norm taken over H*d instead of per head."""
    rng = np.random.default_rng(7)
    B, T, H, d, K = 1, 9, 3, 8, 4
    xs = [rng.standard_normal((B, T, H * d)) * (1.0 + 2.0 * n) for n in range(3)]
    ws = [rng.standard_normal((K, H * d)) for _ in range(3)]
    q, k, v, _ = Lr.prologue(*xs, *ws, H)
    for n, got in enumerate((q, k, v)):
        s = _indep_swish_conv(xs[n][0], ws[n]).reshape(T, H, d)
        if n < 2:
            nrm = np.linalg.norm(s, axis=-1, keepdims=True)
            np.testing.assert_allclose(got[0], s / (nrm + 1e-12), rtol=1e-12, atol=1e-14)
            np.testing.assert_allclose(np.linalg.norm(got[0], axis=-1), 1.0, rtol=1e-10)
        else:
            np.testing.assert_allclose(got[0], s, rtol=1e-12, atol=1e-14)
            assert np.max(np.abs(np.linalg.norm(got[0], axis=-1) - 1.0)) > 0.1


def test_l2_eps_is_added_to_the_norm_not_under_the_root():
    """x / (||x|| + 1e-12) (net/norm.py:53-66): a row of norm 1e-12 comes out
    with norm 1/2; x / sqrt(||x||^2 + 1e-12) would give ~1e-6."""
    x = np.zeros((2, 16))
    x[0, 3] = 1e-12
    x[1, :4] = 0.5e-12
    np.testing.assert_allclose(np.linalg.norm(Lr.l2_norm(x), axis=-1), 0.5, rtol=1e-12)


def test_epilogue_rms_eps_sigmoid_gate_and_per_head_norm():
    """y = sigmoid(z) * o / sqrt(mean_head(o^2) + 1e-6) (net/kda.py:205-214,
    net/norm.py:69-73): per-head RMS of y equals sigmoid(z) for o >> eps; a
    head with mean(o^2) = 1e-6 is divided by sqrt(2e-6) (eps under the root,
    added to the mean, not to the sum); the gate multiplies after the norm."""
    rng = np.random.default_rng(8)
    B, T, H, dv = 1, 3, 2, 16
    o = rng.standard_normal((B, T, H, dv))
    o[:, :, 1] *= 100.0                                  # heads on different scales
    z = np.zeros((B, T, H * dv))
    y = Lr.epilogue(o, z).reshape(B, T, H, dv)
    rms = np.sqrt(np.mean(y * y, axis=-1))
    np.testing.assert_allclose(rms, 0.5, rtol=1e-5)      # sigmoid(0) = 1/2
    tiny = np.full((1, 1, 1, dv), 1e-3)                  # mean(o^2) = 1e-6
    yt = Lr.epilogue(tiny, np.full((1, 1, dv), 50.0))    # sigmoid(50) = 1 in fp64 to 2e-22
    np.testing.assert_allclose(yt, 1e-3 / np.sqrt(2e-6), rtol=1e-12)
    zz = rng.standard_normal((B, T, H * dv))
    from scipy.special import expit
    np.testing.assert_allclose(Lr.epilogue(o, zz), expit(zz) * Lr.epilogue(o, np.full_like(zz, 50.0)),
                               rtol=1e-12)


def _prologue_variant(variant):
    def prologue(qp, kp, vp, wq, wk, wv, H, bufs=None):
        outs = []
        for n, (x, w) in enumerate(((qp, wq), (kp, wk), (vp, wv))):
            x = np.asarray(x, np.float64)
            B, T, HD = x.shape
            y = np.stack([Lr.short_conv(x[b], w)[0] for b in range(B)])
            if variant == "l2_before_swish" and n < 2:
                y = Lr.swish(Lr.l2_norm(y.reshape(B, T, H, HD // H)))
            else:
                y = Lr.swish(y).reshape(B, T, H, HD // H)
                if n < 2 or variant == "v_normalised":
                    y = Lr.l2_norm(y)
                if variant == "norm_over_all_heads" and n < 2:
                    s = Lr.swish(np.stack([Lr.short_conv(x[b], w)[0] for b in range(B)]))
                    y = (s / (np.linalg.norm(s, axis=-1, keepdims=True) + 1e-12)).reshape(B, T, H, HD // H)
            outs.append(y)
        return outs[0], outs[1], outs[2], None
    return prologue


@pytest.mark.parametrize("variant", ["l2_before_swish", "v_normalised", "norm_over_all_heads"])
def test_mutated_prologue_is_caught(monkeypatch, variant):
    monkeypatch.setattr(Lr, "prologue", _prologue_variant(variant))
    with pytest.raises(AssertionError):
        test_prologue_order_conv_swish_then_l2_on_q_k_only()


def test_mutated_l2_eps_is_caught(monkeypatch):
    monkeypatch.setattr(Lr, "l2_norm", lambda x, eps=1e-12: x / np.sqrt(np.sum(x * x, -1, keepdims=True) + eps))
    with pytest.raises(AssertionError):
        test_l2_eps_is_added_to_the_norm_not_under_the_root()


@pytest.mark.parametrize("variant", ["eps_outside_root", "eps_on_sum", "gate_before_norm"])
def test_mutated_epilogue_is_caught(monkeypatch, variant):
    def epilogue(o, gate_logits, eps=1e-6):
        o = np.asarray(o, np.float64)
        B, T, H, dv = o.shape
        g = 1.0 / (1.0 + np.exp(-np.asarray(gate_logits, np.float64))).reshape(B, T, H, dv)
        if variant == "eps_outside_root":
            y = o / (np.sqrt(np.mean(o * o, -1, keepdims=True)) + eps)
        elif variant == "eps_on_sum":
            y = o * np.sqrt(dv) / np.sqrt(np.sum(o * o, -1, keepdims=True) + eps)
        else:
            go = g * o
            return Lr.headwise_rms_norm(go, eps).reshape(B, T, H * dv)
        return (g * y).reshape(B, T, H * dv)
    monkeypatch.setattr(Lr, "epilogue", epilogue)
    with pytest.raises(AssertionError):
        test_epilogue_rms_eps_sigmoid_gate_and_per_head_norm()
