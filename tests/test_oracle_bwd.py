"""Pins of the oracle's chunked backward (no GPU).

``oracle.kda_oracle.chunk_bwd`` transcribes the reference's analytic adjoint
(``net/kernels/kda_cc_fused_bwd.py:30-55``) and its reverse scan
(``net/kernels/kda_cc_fused_persist.py:794-842``).  Nothing here retypes
those equations: the gradients are checked against

* central finite differences of the oracle's chunked *forward* (float64),
  along random directions and element by element on a tiny case (the
  reference pins its adjoint the same way, fp64 FD below 1e-6,
  ``net/tests/test_kda_chunked_cc.py:364``);
* torch autograd through an independent token-by-token recurrence written
  below (the delta rule ``net/kda.py:298-310``, ``o = S^T q`` ``:293``);
* the reference's planted-mistake discipline: a copy of the adjoint with a
  dropped term fails the FD pin.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import inputs, kda_oracle as K

NAMES = ("q", "k", "v", "g", "beta", "h0")


def _case(B, T, H, dk, dv, seed):
    d = inputs.make_inputs(B, T, H, dk, dv, seed=seed, dtype="fp32", h0_std=0.3)
    rng = np.random.default_rng(seed + 100)
    do = rng.standard_normal((B, T, H, dv))
    dht = rng.standard_normal((B, H, dk, dv))
    return {n: d[n].astype(np.float64) for n in NAMES}, do, dht


def _loss(x, do, dht, C, scale=1.0):
    o, ht = K.chunk_fwd(x["q"], x["k"], x["v"], x["g"], x["beta"], h0=x["h0"], chunk=C, scale=scale)
    return float((o.numpy() * do).sum() + (ht.numpy() * dht).sum())


def _grads(x, do, dht, C, scale=1.0):
    dq, dk, dv, dg, db, dh0 = K.chunk_bwd(x["q"], x["k"], x["v"], x["g"], x["beta"], do, dht=dht,
                                          h0=x["h0"], chunk=C, scale=scale)
    return dict(q=dq, k=dk, v=dv, g=dg, beta=db, h0=dh0)


@pytest.mark.parametrize("T,C,scale", [(21, 8, 1.0), (32, 16, 1.0), (19, 16, 0.7)])
def test_directional_derivatives_match_finite_differences(T, C, scale):
    x, do, dht = _case(1, T, 2, 6, 5, seed=T)
    gr = _grads(x, do, dht, C, scale)
    rng = np.random.default_rng(7)
    eps = 1e-6
    for n in NAMES:
        u = rng.standard_normal(x[n].shape)
        xp = dict(x); xp[n] = x[n] + eps * u
        xm = dict(x); xm[n] = x[n] - eps * u
        fd = (_loss(xp, do, dht, C, scale) - _loss(xm, do, dht, C, scale)) / (2 * eps)
        an = float((gr[n] * u).sum())
        assert abs(fd - an) <= 1e-6 * max(1.0, abs(fd)), (n, fd, an)


def test_every_element_matches_finite_differences_tiny():
    x, do, dht = _case(1, 11, 1, 3, 2, seed=5)
    C = 4
    gr = _grads(x, do, dht, C)
    eps = 1e-6
    for n in NAMES:
        flat = x[n].reshape(-1)
        g_an = gr[n].reshape(-1)
        for i in range(flat.size):
            xp = dict(x); a = flat.copy(); a[i] += eps; xp[n] = a.reshape(x[n].shape)
            xm = dict(x); b = flat.copy(); b[i] -= eps; xm[n] = b.reshape(x[n].shape)
            fd = (_loss(xp, do, dht, C) - _loss(xm, do, dht, C)) / (2 * eps)
            assert abs(fd - g_an[i]) <= 1e-6 * max(1.0, abs(fd)), (n, i, fd, g_an[i])


def _recurrent_torch(q, k, v, g, beta, h0):
    """Token-by-token delta rule in torch (autograd-able), [B, T, H, d] inputs."""
    B, T, H, dk = q.shape
    S = h0
    outs = []
    for t in range(T):
        a = torch.exp(g[:, t])                                        # [B, H, dk]
        Sd = a[..., None] * S
        kt, vt, bt = k[:, t], v[:, t], beta[:, t]
        u = torch.einsum("bhd,bhde->bhe", kt, Sd)                     # S~^T k
        S = Sd + bt[..., None, None] * kt[..., None] * (vt - u)[..., None, :]
        outs.append(torch.einsum("bhd,bhde->bhe", q[:, t], S))
    return torch.stack(outs, 1), S


def test_matches_autograd_of_the_recurrence():
    B, T, H, dk, dv = 2, 50, 2, 8, 6
    x, do, dht = _case(B, T, H, dk, dv, seed=11)
    ts = {n: torch.tensor(x[n], dtype=torch.float64, requires_grad=True) for n in NAMES}
    o, ht = _recurrent_torch(ts["q"], ts["k"], ts["v"], ts["g"], ts["beta"], ts["h0"])
    loss = (o * torch.tensor(do)).sum() + (ht * torch.tensor(dht)).sum()
    loss.backward()
    gr = _grads(x, do, dht, C=16)
    for n in NAMES:
        ref = ts[n].grad.numpy()
        err = np.abs(gr[n] - ref).max() / max(np.abs(ref).max(), 1e-30)
        assert err < 1e-9, (n, err)


def test_chunk_size_invariance():
    x, do, dht = _case(1, 40, 2, 8, 8, seed=3)
    a = _grads(x, do, dht, C=8)
    b = _grads(x, do, dht, C=32)
    for n in NAMES:
        np.testing.assert_allclose(a[n], b[n], rtol=1e-9, atol=1e-11)


def test_zero_cotangents_give_zero_gradients():
    x, do, dht = _case(1, 20, 1, 4, 4, seed=2)
    gr = _grads(x, np.zeros_like(do), np.zeros_like(dht), C=8)
    for n in NAMES:
        assert np.abs(gr[n]).max() == 0.0


def test_planted_mistake_fails_the_fd_pin(monkeypatch):
    """A copy of the adjoint without the dY*lam term of dk fails the FD check."""
    x, do, dht = _case(1, 16, 1, 4, 3, seed=9)
    orig = K.chunk_step_bwd

    def broken(q, k, v, G, beta, S, do_, dS_next):
        dq, dk_, dv_, dG, db, dS = orig(q, k, v, G, beta, S, do_, dS_next)
        lam = torch.exp(G[:, -1:, :] - G)
        ar = torch.arange(q.shape[1])
        # recompute v~ to remove the dY * lam contribution
        tril = (ar[:, None] >= ar[None, :]).to(q.dtype)
        E = torch.exp(torch.clamp(G[:, :, None, :] - G[:, None, :, :], max=0.0))
        strict = (ar[:, None] > ar[None, :]).to(q.dtype)
        L = strict * torch.einsum("ncid,ncd,nid->nci", E, k * beta[:, :, None], k)
        SM = torch.linalg.inv(torch.eye(q.shape[1], dtype=q.dtype) + L)
        vt = SM @ (v * beta[:, :, None]) - SM @ (torch.exp(G) * k * beta[:, :, None]) @ S
        dY = vt @ dS_next.transpose(1, 2)
        return dq, dk_ - dY * lam, dv_, dG, db, dS

    monkeypatch.setattr(K, "chunk_step_bwd", broken)
    gr = _grads(x, do, dht, C=8)
    u = np.random.default_rng(1).standard_normal(x["k"].shape)
    eps = 1e-6
    xp = dict(x); xp["k"] = x["k"] + eps * u
    xm = dict(x); xm["k"] = x["k"] - eps * u
    fd = (_loss(xp, do, dht, 8) - _loss(xm, do, dht, 8)) / (2 * eps)
    assert abs(fd - float((gr["k"] * u).sum())) > 1e-4


def test_cc_scan_bwd_matches_finite_differences():
    """The seam's cotangents (dalpha through g = log alpha, dbeta32 through
    the 32-column mean) against central differences of the seam's forward."""
    rng = np.random.default_rng(5)
    T, H, d = 24, 2, 4
    q = rng.standard_normal((T, H * d)) * 0.5
    k = rng.standard_normal((T, H * d)) * 0.5
    v = rng.standard_normal((T, H * d))
    alpha = np.exp(-rng.uniform(0.01, 0.8, (T, H * d)))
    beta32 = rng.uniform(0.1, 0.9, (T, H * 32))          # unequal columns: beta is their mean
    S = rng.standard_normal((H, d, d)) * 0.3
    do = rng.standard_normal((T, H * d))
    dS = rng.standard_normal((H, d, d))
    x = dict(q=q, k=k, v=v, alpha=alpha, beta32=beta32, S=S)

    def loss(y):
        o, sn = K.cc_scan(y["q"], y["k"], y["v"], y["alpha"], y["beta32"], y["S"], chunk=8)
        return float((o * do).sum() + (sn * dS).sum())

    grads = dict(zip(("q", "k", "v", "alpha", "beta32", "S"),
                     K.cc_scan_bwd(q, k, v, alpha, beta32, S, do, dS, chunk=8)))
    eps = 1e-6
    for n in x:
        u = rng.standard_normal(x[n].shape)
        xp = dict(x); xp[n] = x[n] + eps * u
        xm = dict(x); xm[n] = x[n] - eps * u
        fd = (loss(xp) - loss(xm)) / (2 * eps)
        an = float((grads[n] * u).sum())
        assert abs(fd - an) <= 1e-6 * max(1.0, abs(fd)), (n, fd, an)
    # dbeta32 is constant over a head's 32 columns
    db = grads["beta32"].reshape(T, H, 32)
    assert np.array_equal(db, np.repeat(db[..., :1], 32, axis=-1))
