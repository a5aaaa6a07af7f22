"""GPU: the intra-chunk kernel's workspace outputs equal the oracle's per-chunk
intermediates (W, U, Aqk, gamma*q, lambda*k, gamma_C).

The kernels hand these to the state kernel in MFMA fragment order; this test
decodes that order on the host (the layout conventions of
``axiom_amd/csrc/kda_common.h``) so a layout or indexing slip in either kernel
shows up as a named, per-quantity failure instead of a wrong final output.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import axiom_amd
from axiom_amd import kda as kmod
from oracle import inputs, kda_oracle as K
from tests.kda_testutil import to_dev

pytestmark = pytest.mark.gpu

C = 64


def _align(x):
    return (x + 255) // 256 * 256


def ws_offsets(B, T, H, dk, dv, es):
    """Mirror of the C ABI's dense workspace layout (kda_api.hip: ws_layout) for a
    call that runs in one segment (its intra-chunk results fit the segment budget)."""
    units = B * ((T + C - 1) // C)
    ch = units * H
    off, res = 0, {}
    for name, nbytes in (("W", ch * C * dk * es), ("GQ", ch * C * dk * es), ("LK", ch * C * dk * es),
                         ("U", ch * C * dv * es), ("AQ", ch * C * C * es), ("GC", ch * dk * 4),
                         ("status", 4)):
        res[name] = off
        off = _align(off + nbytes)
    res["total"] = off
    return res


def slot_channel(j, gq, e):
    return 32 * j + 4 * gq + (e & 3) + 16 * (e >> 2)


def _lane_grid():
    lane = np.arange(64)
    return lane & 15, lane >> 4


def decode(ws: np.ndarray, B, T, H, dk, dv, es):
    """Decode the fragment-ordered workspace into [B, H, n, ...] arrays."""
    off = ws_offsets(B, T, H, dk, dv, es)
    n = (T + C - 1) // C
    ch = B * n * H
    sdt = np.float32 if es == 4 else np.float16

    def arr(name, count):
        return ws[off[name]: off[name] + count * es].view(sdt).astype(np.float64)

    r, gq = _lane_grid()
    nj = dk // 32
    out = {}
    # W / GQ: [ch][ct][j][lane][8] -> X[c = 16ct + r][d = slot_channel(j, gq, e)]
    for name in ("W", "GQ"):
        raw = arr(name, ch * C * dk).reshape(ch, C // 16, nj, 64, 8)
        X = np.zeros((ch, C, dk))
        for ct in range(C // 16):
            for j in range(nj):
                for e in range(8):
                    X[:, 16 * ct + r, slot_channel(j, gq, e)] = raw[:, ct, j, :, e]
        out[name] = X
    # LK: [ch][dt][jj][lane][8] -> LK[c = slot_channel(jj, gq, e)][d = 16dt + r]
    raw = arr("LK", ch * C * dk).reshape(ch, dk // 16, 2, 64, 8)
    X = np.zeros((ch, C, dk))
    for dt in range(dk // 16):
        for jj in range(2):
            for e in range(8):
                X[:, slot_channel(jj, gq, e), 16 * dt + r] = raw[:, dt, jj, :, e]
    out["LK"] = X
    # U: [ch][ct][et][lane][4] -> U[c = 16ct + 4gq + i][e = 16et + r]
    raw = arr("U", ch * C * dv).reshape(ch, C // 16, dv // 16, 64, 4)
    X = np.zeros((ch, C, dv))
    for ct in range(C // 16):
        for et in range(dv // 16):
            for i in range(4):
                X[:, 16 * ct + 4 * gq + i, 16 * et + r] = raw[:, ct, et, :, i]
    out["U"] = X
    # AQ: [ch][ct][jj][lane][8] -> Aqk[c = 16ct + r][c' = slot_channel(jj, gq, e)]
    raw = arr("AQ", ch * C * C).reshape(ch, C // 16, 2, 64, 8)
    X = np.zeros((ch, C, C))
    for ct in range(C // 16):
        for jj in range(2):
            for e in range(8):
                X[:, 16 * ct + r, slot_channel(jj, gq, e)] = raw[:, ct, jj, :, e]
    out["Aqk"] = X
    out["GC"] = ws[off["GC"]: off["GC"] + ch * dk * 4].view(np.float32).astype(np.float64).reshape(ch, dk)
    # chunk-head index ch = (b * n + chunk) * H + h  ->  [B, H, n, ...]
    for name in out:
        x = out[name]
        out[name] = x.reshape(B, n, H, *x.shape[1:]).swapaxes(1, 2)
    return out


@pytest.mark.parametrize("prec,dk", [("fp32", 64), ("fp32", 128), ("bf16", 64), ("bf16", 128)])
def test_intra_outputs_match_oracle(cuda, prec, dk):
    B, T, H = 1, 128, 2
    d = inputs.make_inputs(B, T, H, dk, dk, seed=31, dtype=prec)
    dt = torch.float32 if prec == "fp32" else torch.bfloat16
    es = 4 if prec == "fp32" else 2
    off = ws_offsets(B, T, H, dk, dk, es)
    assert kmod.chunk_fwd_workspace_bytes(B, T, H, dk, dk, in_code=0 if prec == "fp32" else 1) == off["total"]
    ws = torch.zeros(off["total"], dtype=torch.uint8, device=cuda)
    axiom_amd.kda_chunk_fwd(*(to_dev(d[n], dt, cuda) for n in ("q", "k", "v", "g", "beta")), workspace=ws)
    torch.cuda.synchronize()
    got = decode(ws.cpu().numpy(), B, T, H, dk, dk, es)
    ref = K.chunk_intermediates(d["q"], d["k"], d["v"], d["g"], d["beta"], chunk=C)
    tol = 1e-5 if prec == "fp32" else 3e-3
    failures = []
    for name in ("GC", "GQ", "LK", "Aqk", "U", "W"):
        a, b = got[name], ref[name]
        err = np.abs(a - b).max() / max(np.abs(b).max(), 1e-30)
        if not err <= tol:
            idx = np.unravel_index(np.argmax(np.abs(a - b)), a.shape)
            failures.append(f"{name}: max rel err {err:.3e} at {idx} got {a[idx]:.6g} ref {b[idx]:.6g}")
    assert not failures, "\n".join(failures)
