"""Rounding-point emulator of the HIP chunked backward (TEST INFRASTRUCTURE ONLY).

Reference = romannekrasovaillm/axiom.  The reference pins the storage roundings
of its own backward kernel (bf16 operands, a bf16 carried ``dS``, fp32
reductions: ``net/kernels/kda_cc_fused_persist.py:1005-1013``) with a CPU
emulation, ``_emulate_bf16_bwd`` (``net/tests/test_kda_cc_fused_persist.py:
1015``), swapped in for ``persist.kernel_bwd`` by its tests (``:327-337``).
This module does the same for the gfx950 backward of this repository
(``axiom_amd/csrc/kda_bwd.hip``) with 16-bit inputs: it is the
per-chunk adjoint of ``kda_oracle.chunk_step_bwd`` (``net/kernels/
kda_cc_fused_bwd.py:139-228``) scanned as ``kda_oracle.chunk_bwd`` does
(``net/kernels/kda_cc_fused_persist.py:794-842``), evaluated in float64, with
every value rounded where the kernels store it or hand it to a matrix core in
a 16-bit form that loses bits:

* stored fp16 by the prep kernel: ``gamma q``, ``lambda k``, ``Aqk``,
  ``T = (I+L)^-1`` and ``W``; kept fp32 (unrounded here): ``G``,
  ``gamma_C`` and ``U``;
* forward state scan: ``S`` fp32, stored fp16 for the chunk kernel and handed
  to the ``W S`` product as that fp16 value; ``v~ = U - W S`` stored fp32 and
  handed to the ``(lambda k)^T v~`` state update as fp16;
* reverse scan and chunk kernel: their products run as bf16 hi/lo triples
  (about 2^-16 of each product), modelled as exact; the cotangents ``dS``,
  ``dv~`` and ``do`` are fp32.

``exact=True`` switches every rounding off, and the emulation must then equal
``kda_oracle.chunk_bwd`` to float64 precision (its own pin, with ragged tails,
``h0``, ``dht`` and ``scale``); ``f16`` names the arrays rounded to fp16
(default: the kernels' set; ``"U"`` and ``"VT"``, storing ``U`` and ``v~``
in fp16, are the choices the kernels do not make), so a test can show what
another choice would cost.  Summation order is not modelled, so the emulation predicts the
kernels' error, not their bits.

Pinned in ``tests/test_emulate_bwd.py`` (CPU) and on the GPU in
``tests/test_gpu_bwd.py`` (the kernels' gradients lie within 1e-4 of this
emulation, and within the 1e-3 bf16 bar of the float64 oracle).
"""

from __future__ import annotations

import numpy as np
import torch

F64 = torch.float64

# the arrays the 16-bit backward stores in fp16 (plus the fp16 operands of the
# forward scan's products, "S_op" and "vt_op")
KERNEL_F16 = ("gq", "lk", "aqk", "T", "W", "S", "S_op", "vt_op")


def _f16(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.float16).to(F64)


def emulate_bwd(q, k, v, g, beta, do, dht=None, h0=None, scale: float = 1.0, chunk: int = 64,
                exact: bool = False, f16=KERNEL_F16):
    """Gradients ``(dq, dk, dv, dg, dbeta, dh0)`` of the chunked forward for
    dense ``[B, T, H, d]`` inputs, as ``kda_oracle.chunk_bwd`` returns them,
    with the 16-bit backward's rounding points (none when ``exact``)."""
    names = set(() if exact else f16)

    def rd(name, x):
        return _f16(x) if name in names else x

    q = np.asarray(q) * scale   # (in q's own precision, as kda_oracle.chunk_bwd scales it)
    q, k, v, g, beta, do = (np.asarray(a, np.float64) for a in (q, k, v, g, beta, do))
    B, T, H, dk = q.shape
    dv = v.shape[-1]
    C = chunk
    n = (T + C - 1) // C
    Tp = n * C
    pad = Tp - T

    def prep(x, d):
        t = torch.from_numpy(np.ascontiguousarray(x)).permute(0, 2, 1, 3).reshape(B * H, T, d)
        if pad:
            t = torch.cat([t, torch.zeros((B * H, pad, d), dtype=F64)], 1)
        return t.reshape(B * H, n, C, d)

    qc, kc, vc, doc = prep(q, dk), prep(k, dk), prep(v, dv), prep(do, dv)
    G = torch.cumsum(prep(g, dk), 2)
    bt = torch.from_numpy(np.ascontiguousarray(beta)).permute(0, 2, 1).reshape(B * H, T)
    if pad:
        bt = torch.cat([bt, torch.zeros((B * H, pad), dtype=F64)], 1)
    bc = bt.reshape(B * H, n, C)
    ar = torch.arange(C)
    tril = (ar[:, None] >= ar[None, :]).to(F64)
    strict = (ar[:, None] > ar[None, :]).to(F64)
    eye = torch.eye(C, dtype=F64)

    # prep kernel: per chunk-head intermediates
    P = []
    for i in range(n):
        qq, kk, vv, GG, bb = qc[:, i], kc[:, i], vc[:, i], G[:, i], bc[:, i][:, :, None]
        E = torch.exp(torch.clamp(GG[:, :, None, :] - GG[:, None, :, :], max=0.0))
        aqk = tril * torch.einsum("ncid,ncd,nid->nci", E, qq, kk)
        L = strict * torch.einsum("ncid,ncd,nid->nci", E, kk * bb, kk)
        gam = torch.exp(GG)
        Tm = torch.linalg.inv(eye + L)
        lam = torch.exp(GG[:, -1:, :] - GG)
        P.append(dict(E=E, gam=gam, lam=lam, gc=gam[:, -1, :], aqk=rd("aqk", aqk), T=rd("T", Tm),
                      W=rd("W", Tm @ (gam * kk * bb)), U=rd("U", Tm @ (vv * bb)), gq=rd("gq", gam * qq),
                      lk=rd("lk", lam * kk)))

    # forward state scan: the incoming state and v~ of every chunk
    S = (torch.zeros((B * H, dk, dv), dtype=F64) if h0 is None
         else torch.from_numpy(np.array(h0, np.float64)).reshape(B * H, dk, dv))
    SI, VT = [], []
    for i in range(n):
        p = P[i]
        vt = p["U"] - p["W"] @ rd("S_op", S)
        SI.append(rd("S", S))
        VT.append(rd("VT", vt))
        S = p["gc"][:, :, None] * S + p["lk"].transpose(1, 2) @ rd("vt_op", vt)

    # reverse scan: the state cotangent leaving each chunk, dv~
    dS = (torch.zeros((B * H, dk, dv), dtype=F64) if dht is None
          else torch.from_numpy(np.array(dht, np.float64)).reshape(B * H, dk, dv))
    DS, DVT = [None] * n, [None] * n
    for i in reversed(range(n)):
        p = P[i]
        DS[i] = dS
        dvt = p["lk"] @ dS + p["aqk"].transpose(1, 2) @ doc[:, i]
        DVT[i] = dvt
        dS = p["gc"][:, :, None] * dS + p["gq"].transpose(1, 2) @ doc[:, i] - p["W"].transpose(1, 2) @ dvt
    dh0 = dS

    # chunk kernel: the rest of the adjoint per chunk
    outs = {x: torch.zeros((B * H, n, C, dk if x != "dv" else dv), dtype=F64) for x in ("dq", "dk", "dv", "dg")}
    dbeta = torch.zeros((B * H, n, C), dtype=F64)
    for i in range(n):
        p = P[i]
        qq, kk, vv = qc[:, i], kc[:, i], vc[:, i]
        b = bc[:, i][:, :, None]
        S_in, vt, dSn, dvt, do_ = SI[i], VT[i], DS[i], DVT[i], doc[:, i]
        gam, lam, E = p["gam"], p["lam"], p["E"]
        dgc = (S_in * dSn).sum(-1)
        dY = vt @ dSn.transpose(1, 2)
        daqk = (do_ @ vt.transpose(1, 2)) * tril
        dgq = do_ @ S_in.transpose(1, 2)
        dq = dgq * gam
        dgamma = dgq * qq
        dW = -(dvt @ S_in.transpose(1, 2))
        Yw = p["T"].transpose(1, 2) @ dW
        Yu = p["T"].transpose(1, 2) @ dvt
        dL = -(Yw @ p["W"].transpose(1, 2) + Yu @ p["U"].transpose(1, 2)) * strict
        dgamma = dgamma + Yw * (kk * b)
        dk_ = Yw * (gam * b)
        dv_ = Yu * b
        db = (Yw * gam * kk).sum(-1) + (Yu * vv).sum(-1)
        dr_a = torch.einsum("nci,ncid,nid->ncd", daqk, E, kk)
        dc_a = torch.einsum("nci,ncid,ncd->nid", daqk, E, qq)
        dq = dq + dr_a
        dk_ = dk_ + dc_a
        dr_k = torch.einsum("nci,ncid,nid->ncd", dL, E, kk)
        dc_k = torch.einsum("nci,ncid,ncd->nid", dL, E, kk * b)
        dk_ = dk_ + dr_k * b + dc_k
        db = db + (dr_k * kk).sum(-1)
        dG = (dr_a * qq - dc_a * kk) + (dr_k * (kk * b) - dc_k * kk) + dgamma * gam
        dk_ = dk_ + dY * lam
        dz = dY * kk * lam
        dG = dG - dz
        dG[:, -1, :] += dz.sum(1) + p["gc"] * dgc
        outs["dq"][:, i] = dq * scale
        outs["dk"][:, i] = dk_
        outs["dv"][:, i] = dv_
        outs["dg"][:, i] = torch.flip(torch.cumsum(torch.flip(dG, [1]), 1), [1])
        dbeta[:, i] = db

    def back(t, d):
        return t.reshape(B, H, Tp, d)[:, :, :T].permute(0, 2, 1, 3).contiguous().numpy()

    return (back(outs["dq"], dk), back(outs["dk"], dk), back(outs["dv"], dv), back(outs["dg"], dk),
            dbeta.reshape(B, H, Tp)[:, :, :T].permute(0, 2, 1).contiguous().numpy(),
            dh0.reshape(B, H, dk, dv).numpy())
