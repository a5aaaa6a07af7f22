"""CPU restatement of the KDA layer's prologue and epilogue (TEST INFRASTRUCTURE ONLY).

Reference = romannekrasovaillm/axiom.  numpy float64.

* ``short_conv`` -- causal depthwise convolution, ``net/shortconv.py:14-33``:
  ``out[t] = sum_i w[i] x[t - i]`` with ``x[t < 0]`` taken from a history
  buffer (zeros when absent), as ``_short_conv_chunk`` ``net/kda.py:383-389``
  prepends the carried buffer; ``short_conv_step`` -- the streaming form,
  ``net/shortconv.py:36-62``.
* ``swish`` ``net/norm.py:15-17``; ``l2_norm`` ``x / (||x|| + 1e-12)``
  ``net/norm.py:53-66``; ``headwise_rms_norm`` ``net/norm.py:69-73``.
* ``prologue`` -- ``net/kda.py:194-202`` (``_postprocess``) after the convs;
  ``epilogue`` -- ``net/kda.py:205-214`` (``_output_gate``) without ``W_o``,
  with the gate given as logits (``gate = sigmoid(W_g x)``, ``:181-183``).

* ``prologue_bwd`` / ``epilogue_bwd`` -- their adjoints, written out
  analytically: conv transpose (``dx[t] = sum_i w[i] da[t + i]``, the
  history rows' share going to the incoming buffer), ``dw[i] = sum_t da[t]
  x[t - i]``, swish ``sigma (1 + a (1 - sigma))``, and the L2 norm with the
  reference's convention that its tangent at a zero row is zero
  (``net/norm.py:53-66`` after the fix pinned by
  ``net/tests/test_22_l2norm_padding_gradient.py``).

Pinned in ``tests/test_layer_oracle.py``: the sequence and streaming convs
agree; the conv equals ``numpy.convolve`` per channel; segment continuation
through the buffer equals one run; L2 and RMS closed forms; the adjoints
against central finite differences of the forward functions, and the zero
row's gradient.
"""

from __future__ import annotations

import numpy as np


def short_conv(x, w, buf=None):
    """x (T, D), w (K, D), buf (K-1, D) or None -> (out (T, D), new_buf (K-1, D))."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    K = w.shape[0]
    hist = np.zeros((K - 1, x.shape[1])) if buf is None else np.asarray(buf, np.float64)
    full = np.concatenate([hist, x], axis=0)
    T = x.shape[0]
    out = np.zeros_like(x)
    for i in range(K):
        out += w[i][None, :] * full[K - 1 - i: K - 1 - i + T]
    return out, full[T:]


def short_conv_step(x_t, w, buf):
    """One token of the streaming conv (``net/shortconv.py:36-62``)."""
    w = np.asarray(w, np.float64)
    K = w.shape[0]
    if K == 1:
        return w[0] * x_t, buf
    hist = np.einsum("kd,kd->d", w[:0:-1], buf)
    return w[0] * x_t + hist, np.concatenate([buf[1:], np.asarray(x_t)[None, :]], axis=0)


def swish(x):
    return x / (1.0 + np.exp(-x))


def l2_norm(x, eps=1e-12):
    return x / (np.linalg.norm(x, axis=-1, keepdims=True) + eps)


def headwise_rms_norm(x, eps=1e-6):
    return x / np.sqrt(np.mean(np.square(x), axis=-1, keepdims=True) + eps)


def prologue(qp, kp, vp, wq, wk, wv, H, bufs=None):
    """[B, T, H*d] projections -> (q, k, v [B, T, H, d], new buffers (3 x [B, K-1, H*d]))."""
    outs, new = [], []
    for n, (x, w) in enumerate(((qp, wq), (kp, wk), (vp, wv))):
        x = np.asarray(x, np.float64)
        B, T, HD = x.shape
        y = np.zeros((B, T, HD))
        nb = []
        for b in range(B):
            hist = None if bufs is None else bufs[n][b]
            y[b], nbuf = short_conv(x[b], w, hist)
            nb.append(nbuf)
        y = swish(y).reshape(B, T, H, HD // H)
        if n < 2:
            y = l2_norm(y)
        outs.append(y)
        new.append(np.stack(nb))
    return outs[0], outs[1], outs[2], new


def epilogue(o, gate_logits, eps=1e-6):
    """o [B, T, H, dv], gate logits [B, T, H*dv] -> [B, T, H*dv]."""
    o = np.asarray(o, np.float64)
    B, T, H, dv = o.shape
    g = 1.0 / (1.0 + np.exp(-np.asarray(gate_logits, np.float64)))
    return g * headwise_rms_norm(o, eps).reshape(B, T, H * dv)


def l2_norm_bwd(x, dy, eps=1e-12):
    """Adjoint of ``l2_norm`` over the last axis; zero on rows with ``||x|| == 0``."""
    x = np.asarray(x, np.float64)
    dy = np.asarray(dy, np.float64)
    n = np.linalg.norm(x, axis=-1, keepdims=True)
    npe = n + eps
    dot = np.sum(x * dy, axis=-1, keepdims=True)
    with np.errstate(divide="ignore", invalid="ignore"):
        dx = dy / npe - x * dot / (np.where(n > 0, n, 1.0) * npe * npe)
    return np.where(n > 0, dx, 0.0)


def swish_bwd(a, ds):
    sg = 1.0 / (1.0 + np.exp(-np.asarray(a, np.float64)))
    return np.asarray(ds, np.float64) * sg * (1.0 + a * (1.0 - sg))


def short_conv_bwd(x, w, da, buf=None):
    """Adjoint of ``short_conv`` for one sequence: (dx (T, D), dw (K, D), dbuf (K-1, D))."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    da = np.asarray(da, np.float64)
    K = w.shape[0]
    T = x.shape[0]
    hist = np.zeros((K - 1, x.shape[1])) if buf is None else np.asarray(buf, np.float64)
    full = np.concatenate([hist, x], axis=0)          # row t of x is row K-1+t of full
    dfull = np.zeros_like(full)
    dw = np.zeros_like(w)
    for i in range(K):
        # out[t] += w[i] full[K-1-i+t]
        dfull[K - 1 - i: K - 1 - i + T] += w[i][None, :] * da
        dw[i] = np.sum(da * full[K - 1 - i: K - 1 - i + T], axis=0)
    return dfull[K - 1:], dw, dfull[:K - 1]


def prologue_bwd(qp, kp, vp, wq, wk, wv, H, dq, dk, dv, bufs=None):
    """Cotangents of ``prologue``: given dq, dk, dv [B, T, H, d] returns
    (dqp, dkp, dvp [B, T, H*d], (dwq, dwk, dwv) [K, H*d], dbufs 3 x [B, K-1, H*d])."""
    dxs, dws, dbs = [], [], []
    for n, (x, w, dy) in enumerate(((qp, wq, dq), (kp, wk, dk), (vp, wv, dv))):
        x = np.asarray(x, np.float64)
        B, T, HD = x.shape
        d = HD // H
        a = np.zeros((B, T, HD))
        for b in range(B):
            a[b], _ = short_conv(x[b], w, None if bufs is None else bufs[n][b])
        s = swish(a)
        dy = np.asarray(dy, np.float64).reshape(B, T, H, d)
        ds = l2_norm_bwd(s.reshape(B, T, H, d), dy) if n < 2 else dy
        da = swish_bwd(a, ds.reshape(B, T, HD))
        dx = np.zeros_like(x)
        dw = np.zeros_like(np.asarray(w, np.float64))
        db = np.zeros((B, w.shape[0] - 1, HD))
        for b in range(B):
            dx[b], dwb, db[b] = short_conv_bwd(x[b], w, da[b], None if bufs is None else bufs[n][b])
            dw += dwb
        dxs.append(dx)
        dws.append(dw)
        dbs.append(db)
    return dxs[0], dxs[1], dxs[2], tuple(dws), dbs


def epilogue_bwd(o, gate_logits, dy, eps=1e-6):
    """Cotangents of ``epilogue``: (do [B, T, H, dv], dgate_logits [B, T, H*dv])."""
    o = np.asarray(o, np.float64)
    B, T, H, dv = o.shape
    z = np.asarray(gate_logits, np.float64).reshape(B, T, H, dv)
    dy = np.asarray(dy, np.float64).reshape(B, T, H, dv)
    sg = 1.0 / (1.0 + np.exp(-z))
    r = 1.0 / np.sqrt(np.mean(o * o, axis=-1, keepdims=True) + eps)
    dz = dy * o * r * sg * (1.0 - sg)
    do = sg * r * dy - o * r ** 3 / dv * np.sum(dy * sg * o, axis=-1, keepdims=True)
    return do, dz.reshape(B, T, H * dv)
