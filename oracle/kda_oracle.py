"""CPU restatement of the reference KDA algebra (TEST INFRASTRUCTURE ONLY).

Reference = romannekrasovaillm/axiom.  Notation per head: chunk length ``C``,
``g = log(alpha) <= 0`` per channel, ``G = cumsum_c(g)`` (inclusive),
``gamma = exp(G)``, ``beta in (0, 1)``.

Functions and what each restates
--------------------------------
``recurrent_fwd`` / ``decode_step`` (numpy, float64)
    The delta rule of ``net/kda.py:298-310`` (``_delta_step``):
    ``S <- (I - beta k k^T) Diag(alpha) S + beta k v^T`` with the read taken
    against ``Diag(alpha) S``, and the output ``o = S^T q`` of ``net/kda.py:293``.
    This is the ground truth every other form is checked against.
``cc_scores``
    Tile-wise decay-weighted scores, ``net/kda.py:588-631`` (``_cc_scores``),
    tile width rule ``net/kda.py:570-585`` (``_cc_tile``: 16 at ``g_min = -5``).
``ut_solve``
    ``(I + L)^{-1}`` as an explicit inverse, ``net/kda.py:434-438``
    (``_solve_pair_jax``).
``chunk_fwd`` (torch CPU, float64 or float32)
    The chunk body ``cc_chunk_step`` core, ``net/kda.py:669-702``: scores,
    ``L = beta * Akk``, ``W = T(beta gamma k)``, ``U = T(beta v)``,
    ``v~ = U - W S``, ``o = (gamma q) S + Aqk v~``,
    ``S' = gamma_C S + (lambda k)^T v~``; scanned over chunks as
    ``net/kda.py:924`` and batched over (B, H) as ``net/model.py:341``.
    Padding of a ragged tail follows ``net/kda.py:829-831`` in spirit (zero
    k/v/q rows) with ``g = 0, beta = 0`` so padded rows leave the state alone;
    the returned final state is the state after the last real token, which is
    what the recurrence defines.  ``cu_seqlens`` (absent in the reference) is
    defined by the invariant "packed run == independent per-sequence runs".

How each is pinned (tests/test_oracle.py)
----------------------------------------
* recurrence: closed forms (beta=0 decay-only, g=0 & beta=0 identity,
  alpha->0 overwrite, single token from S0=0 gives ``o = beta (k.q) v``,
  orthonormal keys with beta=1 store ``S^T k_i = v_i`` exactly) and a scalar
  brute-force loop on tiny inputs;
* chunked form: equals the recurrence within 1e-4 for C in {16, 32, 64, 128}
  (the reference's own bar, ``net/tests/test_kda_chunked_cc.py:189-208``),
  chunk-size invariance, per-chunk states, T < C and ragged tails
  (``net/tests/test_kda_chunked_cc.py:270-288``, ``:413-427``);
* scores: brute-force ``(C, C, dk)`` decay-ratio tensor
  (``net/tests/test_kda_chunked_cc.py:221-247``);
* UT solve: ``scipy.linalg.solve_triangular(unit_diagonal=True)`` and the
  Neumann product identity (``net/kernels/kda_ut_solve.py:20-27``);
* varlen: packed == per-sequence; decode: T decode steps == chunked forward.
* ``chunk_intermediates``: the per-chunk W, U, Aqk, gamma*q, lambda*k and
  gamma_C alone rebuild o and the final state of the token recurrence (fp64,
  1e-10, ragged tail and h0 included), ``T (I + L) = I`` with ``L`` built by
  brute force from its definition, and planted slips (lambda*k transposed,
  an exclusive gamma, a strict Aqk, W without beta, gamma_C of one row, U of
  the wrong chunk) each fail the rebuild.
* ``cc_tile``: the values of ``net/kda.py:577-585`` (16 at ``g_min = -5``,
  8 at -10, 16 at 0, ...) and the rule they follow (the widest tile <= 16
  with ``tile * |g_min| <= 80``).
* ``cc_scan`` / ``cc_scan_bwd`` (the seam's operands: alpha, beta32 as a
  32-column mean): the backward against central finite differences of the
  forward in every input, with unequal beta32 columns (tests/test_oracle_bwd.py).
* mutation tests plant a dropped term, a sign flip, a transposed operand and an
  off-by-one in the decay into copies of these functions and show that at
  least one pin fails for each.
No function here is "parity unpinned".
"""

from __future__ import annotations

import numpy as np
import torch

# ---------------------------------------------------------------------------
# Recurrent form (ground truth)
# ---------------------------------------------------------------------------


def decode_step(q, k, v, g, beta, S, scale: float = 1.0):
    """One token per chain: ``net/kda.py:298-310`` then ``o = S'^T q`` (``:293``).

    Shapes: ``q, k, g [..., dk]``, ``v [..., dv]``, ``beta [...]``,
    ``S [..., dk, dv]``.  float64 throughout; returns ``(o, S_new)``.
    """
    q = np.asarray(q, np.float64) * scale
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    alpha = np.exp(np.asarray(g, np.float64))
    beta = np.asarray(beta, np.float64)
    S = np.asarray(S, np.float64)
    decayed = alpha[..., :, None] * S                      # Diag(alpha) S
    read = np.einsum("...d,...de->...e", alpha * k, S)     # (alpha*k)^T S
    S_new = decayed + beta[..., None, None] * k[..., :, None] * (v - read)[..., None, :]
    o = np.einsum("...d,...de->...e", q, S_new)            # S'^T q
    return o, S_new


def recurrent_fwd(q, k, v, g, beta, h0=None, cu_seqlens=None, scale: float = 1.0):
    """Token-by-token recurrence over ``[B, T, H, d]`` inputs (float64).

    Returns ``(o [B,T,H,dv], ht [N,H,dk,dv])`` with ``N = B`` or the number of
    sequences when ``cu_seqlens`` is given (then ``B`` must be 1).
    """
    q, k, v, g, beta = (np.asarray(x, np.float64) for x in (q, k, v, g, beta))
    B, T, H, dk = q.shape
    dv = v.shape[-1]
    if cu_seqlens is None:
        S = np.zeros((B, H, dk, dv)) if h0 is None else np.array(h0, np.float64)
        o = np.zeros((B, T, H, dv))
        for t in range(T):
            o[:, t], S = decode_step(q[:, t], k[:, t], v[:, t], g[:, t], beta[:, t], S, scale)
        return o, S
    if B != 1:
        raise ValueError("cu_seqlens requires B == 1")
    cu = np.asarray(cu_seqlens, np.int64)
    n = len(cu) - 1
    o = np.zeros((1, T, H, dv))
    hts = np.zeros((n, H, dk, dv))
    for i in range(n):
        a, b = int(cu[i]), int(cu[i + 1])
        h0_i = None if h0 is None else np.asarray(h0)[i:i + 1]
        o_i, ht_i = recurrent_fwd(q[:, a:b], k[:, a:b], v[:, a:b], g[:, a:b], beta[:, a:b],
                                  h0=h0_i, scale=scale)
        o[:, a:b] = o_i
        hts[i] = ht_i[0]
    return o, hts


# ---------------------------------------------------------------------------
# Chunked WY/UT form (net/kda.py:570-705), torch CPU
# ---------------------------------------------------------------------------


def cc_tile(g_min: float = -5.0) -> int:
    """Row-tile width of the decay factors, ``net/kda.py:577-585``."""
    step = abs(float(g_min))
    cap = int(80.0 / step) if step > 0 else 16
    return max(1, min(16, cap))


def cc_scores(row: torch.Tensor, col: torch.Tensor, G: torch.Tensor, tile: int,
              strict: bool) -> torch.Tensor:
    """``sum_d exp(G_c - G_i) row_c[d] col_i[d]`` masked to ``c >= i`` (``c > i``).

    Restates ``net/kda.py:588-631``: each row tile measures its decay against
    its own first position ``p``, ``exp(G_c - G_i) = exp(G_c - G_p) exp(G_p - G_i)``.
    ``row, col, G``: ``[N, C, dk]``; returns ``[N, C, C]``.
    """
    N, C, _ = row.shape
    out = torch.zeros((N, C, C), dtype=row.dtype)
    for p in range(0, C, tile):
        b = min(tile, C - p)
        ref = G[:, p:p + 1, :]
        rows = row[:, p:p + b, :] * torch.exp(G[:, p:p + b, :] - ref)
        cols = col[:, :p + b, :] * torch.exp(ref - G[:, :p + b, :])
        blk = rows @ cols.transpose(1, 2)
        ri = torch.arange(p, p + b)[:, None]
        ci = torch.arange(p + b)[None, :]
        keep = (ri > ci) if strict else (ri >= ci)
        out[:, p:p + b, :p + b] = torch.where(keep, blk, torch.zeros((), dtype=blk.dtype))
    return out


def ut_solve(L: torch.Tensor) -> torch.Tensor:
    """``T = (I + L)^{-1}`` for strictly-lower ``L [N, C, C]`` (``net/kda.py:434-438``)."""
    C = L.shape[-1]
    eye = torch.eye(C, dtype=L.dtype).expand_as(L)
    return torch.linalg.inv(eye + L)


def chunk_step(q, k, v, G, beta, S, tile: int = 16):
    """One chunk for ``N`` chains: ``net/kda.py:669-702``.

    ``q, k, G [N, C, dk]``, ``v [N, C, dv]``, ``beta [N, C]``, ``S [N, dk, dv]``
    (``G`` is the in-chunk inclusive cumsum of ``g``).  Returns ``(o, S_new)``.
    """
    aqk = cc_scores(q, k, G, tile, strict=False)                  # :677
    akk = cc_scores(k, k, G, tile, strict=True)                   # :678
    L = akk * beta[:, :, None]                                    # :681
    gamma = torch.exp(G)                                          # :684
    xw = gamma * k * beta[:, :, None]                             # :685
    vw = v * beta[:, :, None]                                     # :686
    Tm = ut_solve(L)                                              # :687
    w = Tm @ xw
    u = Tm @ vw
    v_tilde = u - w @ S                                           # :690
    o = (gamma * q) @ S + aqk @ v_tilde                           # :693-696
    G_last = G[:, -1:, :]
    lam = torch.exp(torch.clamp(G_last - G, max=0.0))             # :700
    S_new = gamma[:, -1, :, None] * S + (lam * k).transpose(1, 2) @ v_tilde   # :701-702
    return o, S_new


def _to_torch(x, dtype):
    return torch.as_tensor(np.ascontiguousarray(x)).to(dtype)


def _chunk_fwd_dense(q, k, v, g, beta, h0, C, tile, dtype, scale, return_chunk_states=False):
    """Chunked forward for equal-length chains: inputs ``[B, T, H, d]`` numpy."""
    B, T, H, dk = q.shape
    dv = v.shape[-1]
    n_chunks = (T + C - 1) // C
    Tp = n_chunks * C
    pad = Tp - T

    def prep(x, d):
        t = _to_torch(x, dtype).permute(0, 2, 1, 3).reshape(B * H, T, d)
        if pad:
            t = torch.cat([t, torch.zeros((B * H, pad, d), dtype=dtype)], dim=1)
        return t.reshape(B * H, n_chunks, C, d)

    qc = prep(np.asarray(q) * scale, dk)
    kc = prep(k, dk)
    vc = prep(v, dv)
    gc = prep(g, dk)
    bt = _to_torch(beta, dtype).permute(0, 2, 1).reshape(B * H, T)
    if pad:
        bt = torch.cat([bt, torch.zeros((B * H, pad), dtype=dtype)], dim=1)
    bc = bt.reshape(B * H, n_chunks, C)
    if h0 is None:
        S = torch.zeros((B * H, dk, dv), dtype=dtype)
    else:
        S = _to_torch(h0, dtype).reshape(B * H, dk, dv).clone()
    o = torch.empty((B * H, n_chunks, C, dv), dtype=dtype)
    states = []
    for n in range(n_chunks):                                     # net/kda.py:924 scan
        G = torch.cumsum(gc[:, n], dim=1)                         # net/kda.py:397-399
        if return_chunk_states:
            states.append(S.clone())
        o[:, n], S = chunk_step(qc[:, n], kc[:, n], vc[:, n], G, bc[:, n], S, tile)
    o = o.reshape(B, H, Tp, dv)[:, :, :T].permute(0, 2, 1, 3)
    out = (o.contiguous(), S.reshape(B, H, dk, dv))
    if return_chunk_states:
        out = out + (torch.stack(states, 1).reshape(B, H, n_chunks, dk, dv),)
    return out


def chunk_fwd(q, k, v, g, beta, h0=None, cu_seqlens=None, chunk: int = 64, tile: int = 16,
              dtype=torch.float64, scale: float = 1.0, return_chunk_states: bool = False):
    """Chunked WY/UT forward (``net/kda.py:856-926`` scan of ``cc_chunk_step``).

    Inputs are numpy ``[B, T, H, d]`` (``beta [B, T, H]``), ``h0 [N, H, dk, dv]``
    or None, ``cu_seqlens [N+1]`` or None (then ``B == 1``).  Returns torch
    tensors ``(o [B,T,H,dv], ht [N,H,dk,dv])`` in ``dtype``.
    """
    if cu_seqlens is None:
        return _chunk_fwd_dense(q, k, v, g, beta, h0, chunk, tile, dtype, scale,
                                return_chunk_states)
    B, T, H, dk = q.shape
    dv = v.shape[-1]
    if B != 1:
        raise ValueError("cu_seqlens requires B == 1")
    cu = np.asarray(cu_seqlens, np.int64)
    n = len(cu) - 1
    o = torch.zeros((1, T, H, dv), dtype=dtype)
    hts = torch.zeros((n, H, dk, dv), dtype=dtype)
    for i in range(n):
        a, b = int(cu[i]), int(cu[i + 1])
        if b == a:
            hts[i] = torch.zeros((H, dk, dv), dtype=dtype) if h0 is None else _to_torch(h0[i], dtype)
            continue
        h0_i = None if h0 is None else np.asarray(h0)[i:i + 1]
        o_i, ht_i = _chunk_fwd_dense(q[:, a:b], k[:, a:b], v[:, a:b], g[:, a:b], beta[:, a:b],
                                     h0_i, chunk, tile, dtype, scale)
        o[:, a:b] = o_i
        hts[i] = ht_i[0]
    return o, hts


# ---------------------------------------------------------------------------
# Chunked backward: the analytic adjoint per chunk, scanned in reverse
# ---------------------------------------------------------------------------


def chunk_step_bwd(q, k, v, G, beta, S, do, dS_next):
    """Adjoint of ``chunk_step`` for ``N`` chains, one chunk.

    Transcribes the equations of ``net/kernels/kda_cc_fused_bwd.py:30-55``
    (code ``:139-228``) with the decay written through ``G`` (the in-chunk
    inclusive cumsum of ``g``) instead of ``alpha``: the returned ``dG`` is
    the cotangent of ``G`` (its reverse cumsum is ``dg``, done by the caller).
    Shapes as ``chunk_step``; ``do [N, C, dv]``, ``dS_next [N, dk, dv]``.
    Returns ``(dq, dk, dv, dG, dbeta, dS_in)``.
    """
    N, C, dk = q.shape
    ar = torch.arange(C)
    tril = (ar[:, None] >= ar[None, :]).to(q.dtype)
    strict = (ar[:, None] > ar[None, :]).to(q.dtype)
    b = beta[:, :, None]
    # E[c, i, d] = exp(G_c - G_i), clamped at 0 above the diagonal (masked there)
    E = torch.exp(torch.clamp(G[:, :, None, :] - G[:, None, :, :], max=0.0))
    aqk = tril * torch.einsum("ncid,ncd,nid->nci", E, q, k)
    L = strict * torch.einsum("ncid,ncd,nid->nci", E, k * b, k)
    gamma = torch.exp(G)
    xw = gamma * k * b
    vw = v * b
    SM = torch.linalg.inv(torch.eye(C, dtype=q.dtype) + L)
    W = SM @ xw
    U = SM @ vw
    vt = U - W @ S
    gc = gamma[:, -1, :]                                      # exp(sum_c la)
    lam = torch.exp(G[:, -1:, :] - G)
    y = lam * k

    dS_acc = gc[:, :, None] * dS_next                         # :176-177
    dgc = (S * dS_next).sum(-1)
    dY = vt @ dS_next.transpose(1, 2)                         # :178-180
    dvt = y @ dS_next + aqk.transpose(1, 2) @ do
    daqk = (do @ vt.transpose(1, 2)) * tril
    dS_acc = dS_acc + (gamma * q).transpose(1, 2) @ do        # :181-184
    dgq = do @ S.transpose(1, 2)
    dgamma = dgq * q
    dq = dgq * gamma
    dU = dvt                                                  # :187-196
    dW = -(dvt @ S.transpose(1, 2))
    dS_acc = dS_acc - W.transpose(1, 2) @ dvt
    Yw = SM.transpose(1, 2) @ dW
    Yu = SM.transpose(1, 2) @ dU
    dL = -(Yw @ W.transpose(1, 2) + Yu @ U.transpose(1, 2)) * strict
    dgamma = dgamma + Yw * (k * b)
    dk_ = Yw * (gamma * b)
    dv_ = Yu * b
    db = (Yw * gamma * k).sum(-1) + (Yu * v).sum(-1)
    dr_a = torch.einsum("nci,ncid,nid->ncd", daqk, E, k)      # :199-211
    dc_a = torch.einsum("nci,ncid,ncd->nid", daqk, E, q)
    dq = dq + dr_a
    dk_ = dk_ + dc_a
    dr_k = torch.einsum("nci,ncid,nid->ncd", dL, E, k)
    dc_k = torch.einsum("nci,ncid,ncd->nid", dL, E, k * b)
    dk_ = dk_ + dr_k * b + dc_k
    db = db + (dr_k * k).sum(-1)
    dG = (dr_a * q - dc_a * k) + (dr_k * (k * b) - dc_k * k)
    dG = dG + dgamma * gamma                                  # through exp(G)
    dlam = dY * k                                             # :214-217
    dk_ = dk_ + dY * lam
    dz = dlam * lam                                           # lam = exp(G_C - G)
    dG = dG - dz
    dG[:, -1, :] += dz.sum(1) + gc * dgc                      # G_C = G[C-1] (:218-220)
    return dq, dk_, dv_, dG, db, dS_acc


def chunk_bwd(q, k, v, g, beta, do, dht=None, h0=None, chunk: int = 64, dtype=torch.float64,
              scale: float = 1.0):
    """Gradients of the chunked forward for dense ``[B, T, H, d]`` inputs.

    The reverse scan of ``net/kernels/kda_cc_fused_persist.py:794-842``
    (``reference_bwd_scan``): a forward scan recomputes each chunk's incoming
    state, a reverse scan runs ``chunk_step_bwd`` per chunk and hands the
    state cotangent to the previous chunk.  ``do [B,T,H,dv]`` and ``dht
    [B,H,dk,dv]`` (None = 0) are the cotangents of ``o`` and of the final
    state.  A ragged tail is zero-padded with ``g = 0, beta = 0, do = 0``,
    which leaves every real row's gradient unchanged.  ``scale`` multiplies q
    as in the forward.  Returns numpy float64 ``(dq, dk, dv, dg, dbeta, dh0)``
    in the input layouts (``dg`` is the cotangent of the log-decay ``g``:
    ``dalpha = dg / alpha`` in the reference's ``alpha`` form).
    """
    B, T, H, dk = q.shape
    dv = v.shape[-1]
    C = chunk
    n = (T + C - 1) // C
    Tp = n * C
    pad = Tp - T

    def prep(x, d):
        t = _to_torch(x, dtype).permute(0, 2, 1, 3).reshape(B * H, T, d)
        if pad:
            t = torch.cat([t, torch.zeros((B * H, pad, d), dtype=dtype)], dim=1)
        return t.reshape(B * H, n, C, d)

    qc = prep(np.asarray(q) * scale, dk)
    kc = prep(k, dk)
    vc = prep(v, dv)
    gcs = torch.cumsum(prep(g, dk), dim=2)
    doc = prep(do, dv)
    bt = _to_torch(beta, dtype).permute(0, 2, 1).reshape(B * H, T)
    if pad:
        bt = torch.cat([bt, torch.zeros((B * H, pad), dtype=dtype)], dim=1)
    bc = bt.reshape(B * H, n, C)
    S = (torch.zeros((B * H, dk, dv), dtype=dtype) if h0 is None
         else _to_torch(h0, dtype).reshape(B * H, dk, dv).clone())
    states = []
    for i in range(n):
        states.append(S)
        _, S = chunk_step(qc[:, i], kc[:, i], vc[:, i], gcs[:, i], bc[:, i], S, tile=C)
    dS = (torch.zeros((B * H, dk, dv), dtype=dtype) if dht is None
          else _to_torch(dht, dtype).reshape(B * H, dk, dv))
    outs = {x: torch.zeros((B * H, n, C, d), dtype=dtype)
            for x, d in (("dq", dk), ("dk", dk), ("dv", dv), ("dg", dk))}
    dbeta = torch.zeros((B * H, n, C), dtype=dtype)
    for i in reversed(range(n)):
        dq_, dk_, dv_, dG, db, dS = chunk_step_bwd(qc[:, i], kc[:, i], vc[:, i], gcs[:, i], bc[:, i],
                                                   states[i], doc[:, i], dS)
        outs["dq"][:, i] = dq_ * scale
        outs["dk"][:, i] = dk_
        outs["dv"][:, i] = dv_
        outs["dg"][:, i] = torch.flip(torch.cumsum(torch.flip(dG, [1]), 1), [1])   # G = cumsum(g)
        dbeta[:, i] = db

    def back(t, d):
        return t.reshape(B, H, Tp, d)[:, :, :T].permute(0, 2, 1, 3).contiguous().numpy()

    return (back(outs["dq"], dk), back(outs["dk"], dk), back(outs["dv"], dv), back(outs["dg"], dk),
            dbeta.reshape(B, H, Tp)[:, :, :T].permute(0, 2, 1).contiguous().numpy(),
            dS.reshape(B, H, dk, dv).numpy())


def cc_scan(q, k, v, alpha, beta32, S, chunk: int = 64):
    """The reference seam ``cc_scan`` (``net/kernels/kda_cc_fused_persist.py:920``)
    in its own operands: ``q, k, alpha (T, H*dk)``, ``v (T, H*dv)``, ``beta32
    (T, H*32)`` (beta = the mean of a head's 32 columns, ``:435``), ``S (H, dk,
    dv)``.  ``g = log(alpha)``; returns numpy float64 ``(o (T, H*dv), S_new)``."""
    H, dk, dv = np.asarray(S).shape
    T = np.asarray(q).shape[0]
    g = np.log(np.asarray(alpha, np.float64)).reshape(1, T, H, dk)
    beta = np.asarray(beta32, np.float64).reshape(T, H, 32).mean(-1)[None]
    o, ht = chunk_fwd(np.asarray(q, np.float64).reshape(1, T, H, dk), np.asarray(k, np.float64).reshape(1, T, H, dk),
                      np.asarray(v, np.float64).reshape(1, T, H, dv), g, beta, h0=np.asarray(S, np.float64)[None],
                      chunk=chunk)
    return o.numpy().reshape(T, H * dv), ht.numpy()[0]


def cc_scan_bwd(q, k, v, alpha, beta32, S, do, dS=None, chunk: int = 64):
    """The seam's backward rule (``kernel_bwd``, ``net/kernels/kda_cc_fused_persist.py:1710``;
    cotangent structure of ``net/kernels/kda_cc_fused_bwd.py:228-239``):
    ``(dq, dk, dv, dalpha, dbeta32, dS_in)`` in float64, ``dalpha = dg / alpha``
    and ``dbeta32`` = the beta cotangent / 32 on each column."""
    H, dk, dv = np.asarray(S).shape
    T = np.asarray(q).shape[0]
    alpha = np.asarray(alpha, np.float64)
    g = np.log(alpha).reshape(1, T, H, dk)
    beta = np.asarray(beta32, np.float64).reshape(T, H, 32).mean(-1)[None]
    dq, dk_, dv_, dg, db, dh0 = chunk_bwd(
        np.asarray(q, np.float64).reshape(1, T, H, dk), np.asarray(k, np.float64).reshape(1, T, H, dk),
        np.asarray(v, np.float64).reshape(1, T, H, dv), g, beta, np.asarray(do, np.float64).reshape(1, T, H, dv),
        dht=None if dS is None else np.asarray(dS, np.float64)[None], h0=np.asarray(S, np.float64)[None],
        chunk=chunk)
    dbeta32 = np.repeat(db[0][..., None] / 32.0, 32, axis=-1).reshape(T, H * 32)
    return (dq.reshape(T, H * dk), dk_.reshape(T, H * dk), dv_.reshape(T, H * dv),
            dg.reshape(T, H * dk) / alpha, dbeta32, dh0[0])


def chunk_intermediates(q, k, v, g, beta, chunk: int = 64, tile: int = 16, scale: float = 1.0):
    """Per-chunk intermediates of ``cc_chunk_step`` (``net/kda.py:669-702``), dense inputs.

    Returns a dict of float64 arrays indexed ``[B, H, n_chunks, ...]``:
    ``W [C, dk]``, ``U [C, dv]``, ``Aqk [C, C]``, ``GQ = gamma*q [C, dk]``,
    ``LK = lambda*k [C, dk]``, ``GC = gamma_C [dk]`` and ``T = (I+L)^-1 [C, C]``
    (T depends only on the chunk's own inputs, not on the carried state).
    """
    B, Tn, H, dk = q.shape
    dv = v.shape[-1]
    n = (Tn + chunk - 1) // chunk
    pad = n * chunk - Tn
    dt = torch.float64

    def prep(x, d):
        t = _to_torch(x, dt).permute(0, 2, 1, 3).reshape(B * H, Tn, d)
        if pad:
            t = torch.cat([t, torch.zeros((B * H, pad, d), dtype=dt)], dim=1)
        return t.reshape(B * H, n, chunk, d)

    qc, kc, vc, gc = prep(np.asarray(q) * scale, dk), prep(k, dk), prep(v, dv), prep(g, dk)
    bt = _to_torch(beta, dt).permute(0, 2, 1).reshape(B * H, Tn)
    if pad:
        bt = torch.cat([bt, torch.zeros((B * H, pad), dtype=dt)], dim=1)
    bc = bt.reshape(B * H, n, chunk)
    out = {name: [] for name in ("W", "U", "Aqk", "GQ", "LK", "GC", "T")}
    for i in range(n):
        G = torch.cumsum(gc[:, i], dim=1)
        qq, kk, vv, bb = qc[:, i], kc[:, i], vc[:, i], bc[:, i]
        aqk = cc_scores(qq, kk, G, tile, strict=False)
        L = cc_scores(kk, kk, G, tile, strict=True) * bb[:, :, None]
        gamma = torch.exp(G)
        Tm = ut_solve(L)
        lam = torch.exp(torch.clamp(G[:, -1:, :] - G, max=0.0))
        out["W"].append(Tm @ (gamma * kk * bb[:, :, None]))
        out["U"].append(Tm @ (vv * bb[:, :, None]))
        out["Aqk"].append(aqk)
        out["GQ"].append(gamma * qq)
        out["LK"].append(lam * kk)
        out["GC"].append(gamma[:, -1, :])
        out["T"].append(Tm)
    return {name: torch.stack(vals, 1).reshape(B, H, n, *vals[0].shape[1:]).numpy()
            for name, vals in out.items()}


def decode_steps(q, k, v, g, beta, S, scale: float = 1.0):
    """``steps`` successive decode steps: inputs ``[steps, B, H, d]``, state ``[B,H,dk,dv]``."""
    outs = []
    S = np.asarray(S, np.float64)
    for t in range(q.shape[0]):
        o, S = decode_step(q[t], k[t], v[t], g[t], beta[t], S, scale)
        outs.append(o)
    return np.stack(outs, 0), S


def decode_steps_torch(q, k, v, g, beta, S, scale: float = 1.0):
    """``decode_steps`` for many chains at once: the same equations
    (``net/kda.py:298-310``, ``:293``) as batched float64 torch products on
    the host's threads, for checks that cover every chain of a large decode
    batch.  Inputs ``[steps, ..., d]`` (``beta [steps, ...]``), state
    ``[..., dk, dv]``; returns numpy ``(o [steps, ..., dv], S)``."""
    f64 = torch.float64
    q, k, v, g, beta = (torch.as_tensor(np.asarray(x), dtype=f64) for x in (q, k, v, g, beta))
    S = torch.as_tensor(np.asarray(S), dtype=f64).clone()
    lead = S.shape[:-2]
    dk, dv = S.shape[-2:]
    S = S.reshape(-1, dk, dv)
    outs = []
    for t in range(q.shape[0]):
        qt, kt, vt = q[t].reshape(-1, dk) * scale, k[t].reshape(-1, dk), v[t].reshape(-1, dv)
        alpha = torch.exp(g[t].reshape(-1, dk))
        S.mul_(alpha[:, :, None])                                   # Diag(alpha) S
        read = torch.bmm(kt[:, None, :], S)[:, 0]                   # (alpha*k)^T S = k^T Diag(alpha) S
        S.add_((beta[t].reshape(-1)[:, None, None] * kt[:, :, None]) * (vt - read)[:, None, :])
        outs.append(torch.bmm(qt[:, None, :], S)[:, 0].reshape(*lead, dv))   # S'^T q
    return torch.stack(outs, 0).numpy(), S.reshape(*lead, dk, dv).numpy()


# ---------------------------------------------------------------------------
# Error metrics used by every parity test
# ---------------------------------------------------------------------------


def rel_l2(x, ref) -> float:
    x = np.asarray(x, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.linalg.norm(ref.ravel())
    return float(np.linalg.norm((x - ref).ravel()) / max(den, 1e-30))


def max_abs(x, ref) -> float:
    x = np.asarray(x, np.float64)
    ref = np.asarray(ref, np.float64)
    if x.size == 0:
        return 0.0
    return float(np.max(np.abs(x - ref)))
