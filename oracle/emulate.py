"""Rounding-point emulator of the HIP chunked forward (TEST INFRASTRUCTURE ONLY).

Reference = romannekrasovaillm/axiom.  The reference pins its own kernel's
storage roundings with a CPU emulation of the kernel arithmetic
(``net/tests/test_kda_cc_fused.py:94-185``, ``_emulate_bf16``; the state
rounding of the persistent design ``net/tests/test_kda_cc_fused_persist.py:
170-192``).  This module does the same for the gfx950 kernels of this
repository: it is the chunk body of ``kda_oracle.chunk_step`` (``net/kda.py:
669-702``) evaluated in float64, with every value rounded where the kernels
store or hand it to a matrix core, and every product accumulated as the
kernels do (fp32 accumulation of rounded operands):

* decay: ``g`` in log2 units (fp32), a tile-local inclusive cumsum over 16-row
  tiles (fp32), ``R = 2^Gt``, ``Cf = 2^(D - Gt)`` (fp32; ``D`` = tile total);
* off-diagonal score tiles (r > s): fp16 operands ``k Cf`` and
  ``(k or q) R M_rs`` (``M_rs`` = 2^(totals of the tiles strictly between));
* diagonal score tiles: fp16 operands ``k Cf`` and ``(k or q) R 2^-D`` when
  every channel's tile decay is above 2^-12 and the operands are at most 8
  in magnitude, else a three-term bf16 hi/lo split
  (``hi*hi + hi*lo + lo*hi``); a tile whose decay passes 2^-100 splits each
  pair (c, i) at the highest bit h where c and i differ, through the anchor
  row a = i | (2^h - 1) (``2^(Gt_c - Gt_a) 2^(Gt_a - Gt_i)``, both <= 1), one
  hi/lo product per level;
* ``L = beta Akk`` fp32; ``T = (I+L)^-1``: diagonal 16x16 blocks inverted in
  fp32 and stored fp16, off-diagonal blocks by the blocked recurrence
  ``T_Rs = -T_RR sum_j L_Rj T_js`` on fp16 operands;
* ``W = T fp16(beta gamma k)``, ``U = T fp16(beta v)``, ``gamma q``,
  ``lambda k`` and ``Aqk`` stored fp16, ``gamma_C`` fp32;
* state step: ``S`` fp32, handed to the matrix cores as fp16; ``v~ = U - W S``
  (fp32) handed on as fp16; ``o = (gamma q) S + Aqk v~`` fp32;
  ``S' = gamma_C S + (lambda k)^T v~`` fp32.

``diag="bf16"`` replaces the diagonal tiles' operands by plain bf16 (the
reference kernel's choice), ``diag="fp32"`` keeps them unrounded, and
``exact=True`` switches every rounding off (the emulator must then equal the
float64 oracle: that is its own pin).  Summation order inside a product is
not modelled (fp32 accumulation in a fixed order), so the emulation predicts
the kernel's error level, not its bits.

Pinned in ``tests/test_emulate.py``: ``exact=True`` equals ``chunk_fwd`` to
1e-11 (ordinary, strong and extreme decay, ragged tails, h0); the emulated
error of the fast mode against the float64 oracle on the config
distributions sits in the band the GPU measures; plain-bf16 diagonal tiles
exceed the 1e-3 bar; and on the GPU the kernel's output lies much closer to
the emulation than to the float64 oracle (``tests/test_gpu_emulate.py``).
"""

from __future__ import annotations

import numpy as np
import torch

F64 = torch.float64
LOG2E = 1.4426950408889634


class _Round:
    """Rounding functions of one emulation: identity when exact."""

    def __init__(self, exact: bool):
        self.exact = exact

    def _to(self, x, dt):
        return x if self.exact else x.to(dt).to(F64)

    def h(self, x):      # fp16 operand / storage
        return self._to(x, torch.float16)

    def b(self, x):      # bf16
        return self._to(x, torch.bfloat16)

    def f(self, x):      # fp32
        return self._to(x, torch.float32)

    def mm(self, a, c):  # fp32 accumulation of already rounded operands
        return self.f(a @ c)

    def hilo(self, x):
        """bf16 hi and lo parts of x (x ~ hi + lo)."""
        hi = self.b(x)
        return hi, self.b(x - hi)



def _extreme_diag(rd, kk, qq, gt):
    """Diagonal 16x16 tile of a tile whose decay passes 2^-100, as the intra
    kernel forms it: the pair (c, i), c > i, through the anchor row
    a = i | (2^h - 1) of the highest bit h where c and i differ, with factors
    2^(G_c - G_a) (query row) and 2^(G_a - G_i) (key row), both <= 1; one
    product per level h (and one for the diagonal, factor 1), each kept for
    its own pairs.  Returns the Akk and Aqk blocks [N, 16 (c), 16 (i)]."""
    def prod(bq, a):
        if rd.exact:
            return rd.mm(bq, a.transpose(1, 2))
        ah, al = rd.hilo(a)
        h, l_ = rd.hilo(bq)
        return rd.f(h @ ah.transpose(1, 2) + l_ @ ah.transpose(1, 2) + h @ al.transpose(1, 2))
    c = torch.arange(16)[:, None]
    i = torch.arange(16)[None, :]
    blk_k = torch.zeros(kk.shape[0], 16, 16, dtype=F64)
    blk_q = torch.where((c == i)[None], prod(qq, kk), blk_k)
    for hb in range(4):
        an = torch.tensor([(r & ~((2 << hb) - 1)) | ((1 << hb) - 1) for r in range(16)])
        key = torch.tensor([((r >> hb) & 1) == 0 for r in range(16)])[None, :, None]
        ga = gt[:, an]
        fk = rd.f(torch.exp2(rd.f(ga - gt)))
        fq = rd.f(torch.exp2(rd.f(gt - ga)))
        zero = torch.zeros_like(kk)
        a = torch.where(key, rd.f(kk * fk), zero)
        bk = torch.where(key, zero, rd.f(kk * fq))
        bq = torch.where(key, zero, rd.f(qq * fq))
        keep = ((c > i) & (((c ^ i) >> hb) == 1))[None]
        blk_k = torch.where(keep, prod(bk, a), blk_k)
        blk_q = torch.where(keep, prod(bq, a), blk_q)
    return blk_k, blk_q

def _scores_tile_pair(rd: _Round, row_op, col_op):
    return rd.mm(row_op, col_op.transpose(-1, -2))


def _chunk(rd: _Round, q, k, v, g, beta, S, diag: str):
    """One chunk for N chains: q, k, g [N, 64, dk], v [N, 64, dv], beta [N, 64],
    S [N, dk, dv] fp32 values held in float64.  Returns (o, S_new)."""
    N, C, dk = q.shape
    nt = C // 16
    g2 = rd.f(g * LOG2E)
    # tile-local inclusive scan in the kernel's order: four doubling steps
    # x[c] += x[c - s], s = 1, 2, 4, 8, inside each 16-row tile (fp32)
    Gt = g2.reshape(N, nt, 16, dk).clone()
    for sft in (1, 2, 4, 8):
        sh = torch.zeros_like(Gt)
        sh[:, :, sft:] = Gt[:, :, :-sft]
        Gt = rd.f(Gt + sh)
    Gt = Gt.reshape(N, C, dk)
    D = [Gt[:, 16 * t + 15] for t in range(nt)]      # tile totals [N, dk]
    R = rd.f(torch.exp2(Gt))
    Dfull = torch.cat([D[t][:, None].expand(N, 16, dk) for t in range(nt)], 1)
    Cf = rd.f(torch.exp2(rd.f(Dfull - Gt)))
    kc = rd.f(k * Cf)
    kr = rd.f(k * R)
    qr = rd.f(q * R)

    Akk = torch.zeros(N, C, C, dtype=F64)
    Aqk = torch.zeros(N, C, C, dtype=F64)
    ri = torch.arange(16)[:, None]
    ci = torch.arange(16)[None, :]
    for r in range(nt):
        rows = slice(16 * r, 16 * r + 16)
        for s in range(r):
            cols = slice(16 * s, 16 * s + 16)
            if r - s == 1:
                M = torch.ones(N, dk, dtype=F64)
            elif r - s == 2:
                M = rd.f(torch.exp2(D[r - 1]))
            else:
                M = rd.f(torch.exp2(rd.f(D[r - 1] + D[r - 2])))
            a = rd.h(kc[:, cols])
            Akk[:, rows, cols] = _scores_tile_pair(rd, rd.h(rd.f(kr[:, rows] * M[:, None])), a)
            Aqk[:, rows, cols] = _scores_tile_pair(rd, rd.h(rd.f(qr[:, rows] * M[:, None])), a)
        # diagonal tile; the operand path is chosen per chain (per chunk-head,
        # as each workgroup decides for its own tile)
        Dr = D[r]
        extreme = (Dr < -100).any(1)                                     # [N]
        iD = rd.f(torch.exp2(-Dr))[:, None]
        ad = kc[:, rows]
        bk = rd.f(kr[:, rows] * iD)
        bq = rd.f(qr[:, rows] * iD)
        mx = torch.stack([kc[:, rows].abs().amax((1, 2)), kr[:, rows].abs().amax((1, 2)),
                          qr[:, rows].abs().amax((1, 2))]).amax(0)
        fp16_ok = (~extreme) & (Dr > -12).all(1) & (mx <= 8)             # [N]
        if diag == "fp32" or rd.exact:
            blk_k = rd.mm(bk, ad.transpose(1, 2))
            blk_q = rd.mm(bq, ad.transpose(1, 2))
        elif diag == "bf16":
            blk_k = rd.mm(rd.b(bk), rd.b(ad).transpose(1, 2))
            blk_q = rd.mm(rd.b(bq), rd.b(ad).transpose(1, 2))
        else:
            ah, al = rd.hilo(ad)
            kh, kl = rd.hilo(bk)
            qh, ql = rd.hilo(bq)
            hl_k = rd.f(kh @ ah.transpose(1, 2) + kl @ ah.transpose(1, 2) + kh @ al.transpose(1, 2))
            hl_q = rd.f(qh @ ah.transpose(1, 2) + ql @ ah.transpose(1, 2) + qh @ al.transpose(1, 2))
            f16_k = rd.mm(rd.h(bk), rd.h(ad).transpose(1, 2))
            f16_q = rd.mm(rd.h(bq), rd.h(ad).transpose(1, 2))
            ok = fp16_ok[:, None, None]
            blk_k = torch.where(ok, f16_k, hl_k)
            blk_q = torch.where(ok, f16_q, hl_q)
        if bool(extreme.any()):
            bk_x, bq_x = _extreme_diag(rd, k[:, rows], q[:, rows], Gt[:, rows])
            x_ = extreme[:, None, None]
            blk_k = torch.where(x_, bk_x, blk_k)
            blk_q = torch.where(x_, bq_x, blk_q)
        zero = torch.zeros((), dtype=F64)
        Akk[:, rows, rows] = torch.where(ri > ci, blk_k, zero)
        Aqk[:, rows, rows] = torch.where(ri >= ci, blk_q, zero)

    L = rd.f(Akk * beta[:, :, None])
    # T = (I + L)^-1: fp32 diagonal inverses stored fp16, blocked off-diagonal recurrence
    Tm = torch.zeros(N, C, C, dtype=F64)
    eye16 = torch.eye(16, dtype=F64)
    for r in range(nt):
        sl = slice(16 * r, 16 * r + 16)
        Tm[:, sl, sl] = rd.f(torch.linalg.inv(eye16 + L[:, sl, sl]))
    Th = rd.h(Tm)
    for r in range(1, nt):
        rr = slice(16 * r, 16 * r + 16)
        for s in range(r - 1, -1, -1):
            cs = slice(16 * s, 16 * s + 16)
            X = torch.zeros(N, 16, 16, dtype=F64)
            for j in range(s, r):
                js = slice(16 * j, 16 * j + 16)
                X = X + rd.h(L[:, rr, js]) @ Th[:, js, cs]
            Tm[:, rr, cs] = -rd.mm(Th[:, rr, rr], rd.h(rd.f(X)))
            Th[:, rr, cs] = rd.h(Tm[:, rr, cs])

    # per-tile prefix / suffix decay products: gamma = R 2^pre, lambda = Cf 2^post
    pre = torch.zeros(N, C, dk, dtype=F64)
    post = torch.zeros(N, C, dk, dtype=F64)
    for t in range(nt):
        sl = slice(16 * t, 16 * t + 16)
        p = sum((D[u] for u in range(t)), torch.zeros(N, dk, dtype=F64))
        q_ = sum((D[u] for u in range(t + 1, nt)), torch.zeros(N, dk, dtype=F64))
        pre[:, sl] = rd.f(torch.exp2(rd.f(p)))[:, None]
        post[:, sl] = rd.f(torch.exp2(rd.f(q_)))[:, None]
    bcol = beta[:, :, None]
    bgk = rd.h(rd.f(kr * rd.f(bcol * pre)))
    W = rd.h(rd.mm(Th, bgk))
    U = rd.h(rd.mm(Th, rd.h(rd.f(bcol * v))))
    GQ = rd.h(rd.f(qr * pre))
    LK = rd.h(rd.f(kc * post))
    Aq = rd.h(Aqk)
    GC = rd.f(torch.exp2(rd.f(D[0] + D[1] + D[2] + D[3])))

    # state step
    Sh = rd.h(S)
    vt = rd.f(U - rd.mm(W, Sh))
    vth = rd.h(vt)
    o = rd.f(rd.mm(GQ, Sh) + rd.mm(Aq, vth))
    S_new = rd.f(GC[:, :, None] * S + rd.mm(LK.transpose(1, 2), vth))
    return o, S_new


def emulate_fwd(q, k, v, g, beta, h0=None, scale: float = 1.0, diag: str = "kernel",
                exact: bool = False):
    """Chunked forward of the HIP kernels with their rounding points.

    Dense inputs ``[B, T, H, d]`` (numpy, any float dtype; the values are used
    as given, so pass the bf16-rounded inputs the kernels read), ``h0
    [B, H, dk, dv]`` or None.  C = 64.  Returns float64 torch
    ``(o [B,T,H,dv], ht [B,H,dk,dv])``.
    """
    if diag not in ("kernel", "bf16", "fp32"):
        raise ValueError(f"unknown diagonal mode {diag!r}")
    rd = _Round(exact)
    B, T, H, dk = q.shape
    dv = v.shape[-1]
    C = 64
    n = (T + C - 1) // C
    pad = n * C - T

    def prep(x, d):
        t = torch.as_tensor(np.ascontiguousarray(x)).to(F64).permute(0, 2, 1, 3).reshape(B * H, T, d)
        if pad:
            t = torch.cat([t, torch.zeros(B * H, pad, d, dtype=F64)], 1)
        return t.reshape(B * H, n, C, d)

    qc = prep(np.asarray(q, np.float64), dk)
    if scale != 1.0:
        qc = rd.f(qc * scale)
    kc, vc, gc = prep(k, dk), prep(v, dv), prep(g, dk)
    bt = torch.as_tensor(np.ascontiguousarray(beta)).to(F64).permute(0, 2, 1).reshape(B * H, T)
    if pad:
        bt = torch.cat([bt, torch.zeros(B * H, pad, dtype=F64)], 1)
    bc = bt.reshape(B * H, n, C)
    S = (torch.zeros(B * H, dk, dv, dtype=F64) if h0 is None
         else rd.f(torch.as_tensor(np.asarray(h0)).to(F64).reshape(B * H, dk, dv)))
    o = torch.empty(B * H, n, C, dv, dtype=F64)
    for i in range(n):
        o[:, i], S = _chunk(rd, qc[:, i], kc[:, i], vc[:, i], gc[:, i], bc[:, i], S, diag)
    o = o.reshape(B, H, n * C, dv)[:, :, :T].permute(0, 2, 1, 3).contiguous()
    return o, S.reshape(B, H, dk, dv)
