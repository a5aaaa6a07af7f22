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

Pinned in ``tests/test_layer_oracle.py``: the sequence and streaming convs
agree; the conv equals ``numpy.convolve`` per channel; segment continuation
through the buffer equals one run; L2 and RMS closed forms.
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
