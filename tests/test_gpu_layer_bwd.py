"""GPU parity of the layer's backward: kda_epilogue_bwd and kda_prologue_bwd
against the float64 adjoints of oracle/layer.py (pinned on the CPU against
finite differences in tests/test_layer_oracle.py), and the differentiable
kda_layer (epilogue backward -> chunked backward -> prologue backward, all
HIP) against the oracle's chain on the same inputs.

The kernels compute in fp32 from inputs of either dtype (bf16 inputs are
rounded identically on both sides), so the bar is the fp32 one: relative L2
<= 1e-5 and max-abs <= 1e-5 x max(1, max|reference|) per gradient, except
where a result is emitted in bf16 (relative L2 <= 4e-3, max-abs <= 1e-2 x
max(1, max|reference|)).  The whole-layer gradients pass through the chunked
backward, whose bar is relative L2 <= 1e-4 (tests/test_gpu_bwd.py); with bf16
projections the recomputed q, k, v are bf16 (as the forward's), so that case
is held to relative L2 <= 1e-2 against the oracle that never rounds them.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import inputs, kda_oracle as Ko, layer as Lr

pytestmark = pytest.mark.gpu


def _as(x, dt):
    """The float64 values a tensor of dtype dt holds for the float32 array x."""
    return torch.from_numpy(np.ascontiguousarray(x)).to(dt).double().numpy()


def _close(name, got, ref, rel_tol=1e-5, abs_tol=1e-5):
    got = got.double().cpu().numpy() if isinstance(got, torch.Tensor) else np.asarray(got)
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    assert np.all(np.isfinite(got)), name
    err = np.abs(got - ref)
    scale = max(1.0, float(np.abs(ref).max()) if ref.size else 1.0)
    den = np.linalg.norm(ref)
    rel = np.linalg.norm(got - ref) / den if den > 0 else float(np.linalg.norm(got))
    assert rel <= rel_tol and (err.size == 0 or err.max() <= abs_tol * scale), (
        f"{name}: rel_l2={rel:.3e} max_abs={err.max() if err.size else 0:.3e} scale={scale:.3g}")


@pytest.mark.parametrize("B,T,H,dv,o_dt,g_dt,dy_dt,dg_dt", [
    (2, 37, 3, 128, torch.float32, torch.float32, torch.float32, torch.float32),
    (1, 64, 2, 64, torch.float32, torch.bfloat16, torch.bfloat16, torch.float32),
    (2, 5, 4, 128, torch.bfloat16, torch.bfloat16, torch.float32, torch.bfloat16),
    (1, 1, 1, 64, torch.float32, torch.float32, torch.float32, torch.bfloat16),
])
def test_epilogue_bwd_matches_oracle(cuda, B, T, H, dv, o_dt, g_dt, dy_dt, dg_dt):
    import axiom_amd
    rng = np.random.default_rng(B * 100 + T)
    o = rng.standard_normal((B, T, H, dv)).astype(np.float32)
    z = rng.standard_normal((B, T, H * dv)).astype(np.float32) * 2
    dy = rng.standard_normal((B, T, H * dv)).astype(np.float32)
    do, dz = axiom_amd.kda_epilogue_bwd(torch.from_numpy(o).to(cuda, o_dt), torch.from_numpy(z).to(cuda, g_dt),
                                        torch.from_numpy(dy).to(cuda, dy_dt), eps=1e-6, dgate_dtype=dg_dt)
    torch.cuda.synchronize()
    rdo, rdz = Lr.epilogue_bwd(_as(o, o_dt), _as(z, g_dt), _as(dy, dy_dt), eps=1e-6)
    _close("do", do, rdo)
    if dg_dt == torch.float32:
        _close("dgate", dz, rdz)
    else:
        _close("dgate", dz, rdz, 4e-3, 1e-2)


def _proj(B, T, H, d, K, seed):
    rng = np.random.default_rng(seed)
    xs = [rng.standard_normal((B, T, H * d)).astype(np.float32) for _ in range(3)]
    ws = [(rng.standard_normal((K, H * d)) * 0.4).astype(np.float32) for _ in range(3)]
    bufs = [rng.standard_normal((B, K - 1, H * d)).astype(np.float32) for _ in range(3)]
    dys = [rng.standard_normal((B, T, H, d)).astype(np.float32) for _ in range(3)]
    return xs, ws, bufs, dys


def _prologue_bwd_case(cuda, xs, ws, bufs, dys, H, in_dt, with_buf):
    import axiom_amd
    xs_t = [torch.from_numpy(x).to(cuda, in_dt) for x in xs]
    ws_t = [torch.from_numpy(w).to(cuda) for w in ws]
    st = tuple(torch.from_numpy(b).to(cuda) for b in bufs) if with_buf else None
    dys_t = [torch.from_numpy(y).to(cuda) for y in dys]
    dx, dw, db = axiom_amd.kda_prologue_bwd(*xs_t, *ws_t, *dys_t, conv_state=st)
    torch.cuda.synchronize()
    rdq, rdk, rdv, rdw, rdb = Lr.prologue_bwd(*(_as(x, in_dt) for x in xs), *ws, H, *dys,
                                              bufs=bufs if with_buf else None)
    for n, got, ref in zip(("dqp", "dkp", "dvp"), dx, (rdq, rdk, rdv)):
        _close(n, got, ref)
    for n, got, ref in zip(("dwq", "dwk", "dwv"), dw, rdw):
        _close(n, got, ref)
    K = ws[0].shape[0]
    if with_buf and K > 1:
        for n, got, ref in zip(("dbq", "dbk", "dbv"), db, rdb):
            _close(n, got, ref)
    else:
        assert db is None


@pytest.mark.parametrize("B,T,H,d,K,in_dt,with_buf", [
    (2, 37, 2, 128, 4, torch.float32, True),
    (1, 70, 3, 64, 4, torch.bfloat16, True),
    (2, 5, 2, 128, 1, torch.float32, False),
    (1, 2, 1, 64, 4, torch.float32, True),       # T < K - 1: the sums reach only part of the buffer
    (1, 200, 2, 128, 8, torch.float32, True),
    (2, 16, 2, 64, 6, torch.bfloat16, False),
    (1, 129, 1, 128, 2, torch.bfloat16, True),   # ragged last 64-row group
])
def test_prologue_bwd_matches_oracle(cuda, B, T, H, d, K, in_dt, with_buf):
    xs, ws, bufs, dys = _proj(B, T, H, d, K, seed=T * 11 + K)
    _prologue_bwd_case(cuda, xs, ws, bufs, dys, H, in_dt, with_buf)


def test_prologue_bwd_zero_rows_get_zero_norm_gradient(cuda):
    """Rows whose swish output is all zeros (zero projections through the conv
    window, or a head whose inputs are all zero): the L2 norm's gradient there
    is zero, the reference's convention at the origin."""
    B, T, H, d, K = 2, 48, 2, 64, 4
    xs, ws, bufs, dys = _proj(B, T, H, d, K, seed=3)
    xs[0][0, :10] = 0.0            # q rows 0..9 of sequence 0 (no carried buffer: a = 0 there)
    xs[1][1, :, :d] = 0.0          # k head 0 of sequence 1 at every row
    _prologue_bwd_case(cuda, xs, ws, bufs, dys, H, torch.float32, with_buf=False)
    import axiom_amd
    xs_t = [torch.from_numpy(x).to(cuda) for x in xs]
    ws_t = [torch.from_numpy(w).to(cuda) for w in ws]
    dys_t = [torch.from_numpy(y).to(cuda) for y in dys]
    dx, dw, _ = axiom_amd.kda_prologue_bwd(*xs_t, *ws_t, *dys_t)
    torch.cuda.synchronize()
    # the k head that is zero everywhere passes no gradient to its inputs
    assert torch.count_nonzero(dx[1][1, :, :d]) == 0


def test_prologue_bwd_empty_sequence(cuda):
    import axiom_amd
    B, H, d, K = 2, 2, 64, 4
    xs, ws, bufs, _ = _proj(B, 0, H, d, K, seed=9)
    xs_t = [torch.from_numpy(x).to(cuda) for x in xs]
    ws_t = [torch.from_numpy(w).to(cuda) for w in ws]
    st = tuple(torch.from_numpy(b).to(cuda) for b in bufs)
    dys_t = [torch.zeros((B, 0, H, d), device=cuda) for _ in range(3)]
    dx, dw, db = axiom_amd.kda_prologue_bwd(*xs_t, *ws_t, *dys_t, conv_state=st)
    torch.cuda.synchronize()
    assert all(t.numel() == 0 for t in dx)
    assert all(torch.count_nonzero(t) == 0 for t in dw)
    assert all(torch.count_nonzero(t) == 0 for t in db)


def _layer_ref(xs, ws, bufs, g, beta, z, h0, dy, dht, H, scale, eps, in_dt, g_dt):
    """The oracle's forward and backward of the layer on the GPU's input values."""
    xr = [_as(x, in_dt) for x in xs]
    gr, br = _as(g, g_dt), _as(beta, g_dt)
    zr = _as(z, in_dt)
    q, k, v, _ = Lr.prologue(*xr, *ws, H, bufs=bufs)
    o, _ = Ko.chunk_fwd(q, k, v, gr, br, h0=h0, scale=scale)
    o = o.numpy()
    do, dz = Lr.epilogue_bwd(o, zr, dy, eps=eps)
    dq, dk, dv, dg, dbeta, dh0 = Ko.chunk_bwd(q, k, v, gr, br, do, dht=dht, h0=h0, scale=scale)
    dqp, dkp, dvp, dw, db = Lr.prologue_bwd(*xr, *ws, H, dq, dk, dv, bufs=bufs)
    return dict(dqp=dqp, dkp=dkp, dvp=dvp, dg=dg, dbeta=dbeta, dgate=dz, dwq=dw[0], dwk=dw[1], dwv=dw[2],
                dbq=db[0], dbk=db[1], dbv=db[2], dh0=dh0)


@pytest.mark.parametrize("B,T,H,d,K,prec,carried,gates32", [
    (1, 100, 2, 64, 4, "fp32", True, False),
    (2, 130, 2, 128, 4, "bf16", True, False),
    (1, 70, 1, 64, 6, "bf16", True, False),      # K > 4: the forward's prologue runs as its own pass
    (2, 77, 2, 128, 4, "bf16", False, False),    # no conv buffers, no initial state
    (1, 90, 2, 128, 3, "bf16", True, True),      # bf16 projections with fp32 g and beta
])
def test_layer_autograd_matches_oracle(cuda, B, T, H, d, K, prec, carried, gates32):
    import axiom_amd
    in_dt = torch.float32 if prec == "fp32" else torch.bfloat16
    g_dt = torch.float32 if gates32 else in_dt
    x = inputs.make_inputs(B, T, H, d, d, seed=T + K, dtype="fp32", h0_std=0.05)
    xs, ws, bufs, _ = _proj(B, T, H, d, K, seed=T * 3 + K)
    rng = np.random.default_rng(T)
    z = rng.standard_normal((B, T, H * d)).astype(np.float32)
    dy = rng.standard_normal((B, T, H * d)).astype(np.float32)
    dht = (rng.standard_normal((B, H, d, d)) * 0.1).astype(np.float32)
    scale = d ** -0.5
    eps = 1e-6

    def leaf(a, dt):
        return torch.from_numpy(np.ascontiguousarray(a)).to(cuda, dt).requires_grad_(True)

    xs_t = [leaf(a, in_dt) for a in xs]
    g_t, b_t = leaf(x["g"], g_dt), leaf(x["beta"], g_dt)
    z_t = leaf(z, in_dt)
    ws_t = [leaf(a, torch.float32) for a in ws]
    st = [leaf(a, torch.float32) for a in bufs] if carried else None
    h0_t = leaf(x["h0"], torch.float32) if carried else None
    y, ht = axiom_amd.kda_layer(*xs_t, g_t, b_t, z_t, *ws_t, conv_state=None if st is None else tuple(st),
                                initial_state=h0_t, scale=scale, eps=eps)
    assert y.dtype == in_dt and ht.dtype == torch.float32
    loss = (y.float() * torch.from_numpy(dy).to(cuda)).sum() + (ht * torch.from_numpy(dht).to(cuda)).sum()
    loss.backward()
    torch.cuda.synchronize()
    # y.float()'s VJP hands the layer dy rounded to y's dtype
    ref = _layer_ref(xs, ws, bufs if carried else None, x["g"], x["beta"], z, x["h0"] if carried else None,
                     _as(dy, in_dt), dht.astype(np.float64), H, scale, eps, in_dt, g_dt)
    got = dict(dqp=xs_t[0].grad, dkp=xs_t[1].grad, dvp=xs_t[2].grad, dg=g_t.grad, dbeta=b_t.grad, dgate=z_t.grad,
               dwq=ws_t[0].grad, dwk=ws_t[1].grad, dwv=ws_t[2].grad)
    if carried:
        got.update(dbq=st[0].grad, dbk=st[1].grad, dbv=st[2].grad, dh0=h0_t.grad)
    else:
        for n in ("dbq", "dbk", "dbv", "dh0"):
            ref.pop(n)
    rel, mx = (1e-4, 1e-4) if prec == "fp32" else (1e-2, 5e-2)
    for name, r in ref.items():
        assert got[name] is not None, name
        _close(name, got[name], np.asarray(r), rel, mx)
