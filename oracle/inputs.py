"""Seeded synthetic inputs for the KDA configs (test infrastructure only).

Distributions (the benchmark configs of this path):

* ``q, k = l2norm(N(0,1))`` per head over ``dk`` with ``x / (||x|| + 1e-12)``
  (the reference's ``l2_norm``, ``net/norm.py:20-23``, applied per head as in
  ``net/kda.py:200-201``);
* ``v ~ N(0,1)``;
* ``beta = sigmoid(N(0,1))`` per token-head;
* ``g = -softplus(N(0,1)) * exp(a_h)`` with ``a_h ~ U(-2, 0)`` per head;
* optional initial state ``h0 ~ N(0, h0_std^2)`` in fp32.

All draws come from one ``numpy.random.Generator(PCG64(seed))`` in the fixed
order q, k, v, beta, g, a, h0.  ``dtype="bf16"`` rounds q, k, v, g and beta to
bfloat16 (round-to-nearest-even) and returns the rounded values as float32, so
that the kernel and the oracle consume bit-identical inputs.
"""

from __future__ import annotations

import numpy as np


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest bfloat16 (ties to even); returns float32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32)
    # NaN stays NaN (the rounding above could turn a NaN payload into inf).
    return np.where(np.isnan(x), x, out).reshape(x.shape)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """The uint16 bit patterns of float32 values that are already bf16-exact."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    return (x.view(np.uint32) >> 16).astype(np.uint16)


def l2norm(x: np.ndarray, eps: float = 1e-12) -> np.ndarray:
    """``x / (||x|| + eps)`` over the last axis (``net/norm.py:20-23``)."""
    n = np.sqrt(np.sum(np.square(x, dtype=np.float64), axis=-1, keepdims=True))
    return (x / (n + eps)).astype(x.dtype)


def _softplus(x: np.ndarray) -> np.ndarray:
    return np.logaddexp(np.float32(0.0), x).astype(np.float32)


def _sigmoid(x: np.ndarray) -> np.ndarray:
    return (1.0 / (1.0 + np.exp(-x.astype(np.float64)))).astype(np.float32)


def make_inputs(B: int, T: int, H: int, dk: int, dv: int, seed: int = 0,
                dtype: str = "bf16", h0_std: float = 0.0, n_states: int | None = None):
    """Draw one input set ``[B, T, H, d]`` (row-major, token-major like FLA).

    Returns a dict with float32 arrays ``q, k, g`` ``[B,T,H,dk]``, ``v``
    ``[B,T,H,dv]``, ``beta`` ``[B,T,H]`` and, when ``h0_std > 0``, ``h0``
    ``[n_states or B, H, dk, dv]``.
    """
    rng = np.random.Generator(np.random.PCG64(seed))
    f32 = np.float32
    q = l2norm(rng.standard_normal((B, T, H, dk), dtype=f32))
    k = l2norm(rng.standard_normal((B, T, H, dk), dtype=f32))
    v = rng.standard_normal((B, T, H, dv), dtype=f32)
    beta = _sigmoid(rng.standard_normal((B, T, H), dtype=f32))
    gz = rng.standard_normal((B, T, H, dk), dtype=f32)
    a = rng.uniform(-2.0, 0.0, size=(H,)).astype(f32)
    g = (-_softplus(gz) * np.exp(a)[None, None, :, None]).astype(f32)
    out = dict(q=q, k=k, v=v, g=g, beta=beta)
    if h0_std > 0.0:
        n = B if n_states is None else n_states
        out["h0"] = (rng.standard_normal((n, H, dk, dv), dtype=f32) * f32(h0_std)).astype(f32)
    if dtype == "bf16":
        for name in ("q", "k", "v", "g", "beta"):
            out[name] = bf16_round(out[name])
    elif dtype != "fp32":
        raise ValueError(f"dtype must be 'bf16' or 'fp32', got {dtype!r}")
    return out


def make_varlen_lengths(n_seqs: int, lo: int, hi: int, seed: int) -> np.ndarray:
    """Sequence lengths drawn uniformly from ``[lo, hi]`` (inclusive)."""
    rng = np.random.Generator(np.random.PCG64(seed + 7919))
    return rng.integers(lo, hi + 1, size=n_seqs).astype(np.int64)


def cu_seqlens_from_lengths(lengths) -> np.ndarray:
    """``[0, l0, l0+l1, ...]`` as int32 (the FLA ``cu_seqlens`` convention)."""
    cu = np.zeros(len(lengths) + 1, dtype=np.int64)
    cu[1:] = np.cumsum(np.asarray(lengths, dtype=np.int64))
    return cu.astype(np.int32)


def make_decode_inputs(B: int, H: int, dk: int, dv: int, steps: int, seed: int = 0,
                       dtype: str = "bf16", state_std: float = 0.02):
    """Decode inputs: per-step ``q,k,g [steps,B,H,dk]``, ``v [steps,B,H,dv]``,
    ``beta [steps,B,H]`` and the fp32 state ``S [B,H,dk,dv] ~ N(0, state_std^2)``."""
    d = make_inputs(steps, B, H, dk, dv, seed=seed, dtype=dtype)
    rng = np.random.Generator(np.random.PCG64(seed + 104729))
    S = (rng.standard_normal((B, H, dk, dv), dtype=np.float32) * np.float32(state_std))
    d["S"] = S.astype(np.float32)
    return d
