"""GPU parity of the prologue (short conv, swish, L2 norm) and epilogue (head-wise
RMSNorm x sigmoid gate) against oracle/layer.py on the same inputs.

fp32 in/out: max-abs error <= 1e-5 (fp32 arithmetic on both sides of a
float64 reference).  bf16 projections or outputs: the inputs are rounded
identically on both sides; the bf16 output rounding (2^-9 relative) sets the
bar: relative L2 <= 4e-3, max-abs <= 1e-2.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import layer as Lr

pytestmark = pytest.mark.gpu


def _as(x, dt):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dt).double().numpy()


def _close(got, ref, exact):
    got = got.double().cpu().numpy()
    err = np.abs(got - ref)
    if exact:
        assert err.max() <= 1e-5, err.max()
    else:
        rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
        assert rel <= 4e-3 and err.max() <= 1e-2, (rel, err.max())


def _proj(B, T, H, d, K, seed):
    rng = np.random.default_rng(seed)
    xs = [rng.standard_normal((B, T, H * d)).astype(np.float32) for _ in range(3)]
    ws = [(rng.standard_normal((K, H * d)) * 0.4).astype(np.float32) for _ in range(3)]
    bufs = [rng.standard_normal((B, K - 1, H * d)).astype(np.float32) for _ in range(3)]
    return xs, ws, bufs


@pytest.mark.parametrize("B,T,H,d,K,in_dt,out_dt", [
    (2, 37, 2, 128, 4, torch.float32, torch.float32),
    (1, 64, 3, 64, 4, torch.bfloat16, torch.bfloat16),
    (2, 5, 2, 128, 1, torch.float32, torch.bfloat16),
    (1, 2, 1, 64, 4, torch.float32, torch.float32),     # T < K - 1: buffer shift
])
def test_prologue_matches_oracle(cuda, B, T, H, d, K, in_dt, out_dt):
    import axiom_amd
    xs, ws, bufs = _proj(B, T, H, d, K, seed=T * 7 + K)
    xs_t = [torch.from_numpy(x).to(cuda, in_dt) for x in xs]
    ws_t = [torch.from_numpy(w).to(cuda) for w in ws]
    st = tuple(torch.from_numpy(b).to(cuda) for b in bufs)
    q, k, v, new = axiom_amd.kda_prologue(*xs_t, *ws_t, H, conv_state=st, out_dtype=out_dt)
    torch.cuda.synchronize()
    rq, rk, rv, rnew = Lr.prologue(*(_as(x, in_dt) for x in xs), *ws, H, bufs=bufs)
    exact = in_dt == torch.float32 and out_dt == torch.float32
    for got, ref in ((q, rq), (k, rk), (v, rv)):
        _close(got, ref, exact)
    for got, ref in zip(new, rnew):
        np.testing.assert_allclose(got.cpu().numpy(), ref, rtol=0, atol=0 if in_dt == torch.float32 else 1e-30)


def test_prologue_segments_chain_bitwise_and_in_place_buffers(cuda):
    import axiom_amd
    B, T, H, d, K = 2, 50, 2, 128, 4
    xs, ws, _ = _proj(B, T, H, d, K, seed=5)
    xs_t = [torch.from_numpy(x).to(cuda) for x in xs]
    ws_t = [torch.from_numpy(w).to(cuda) for w in ws]
    q, k, v, st = axiom_amd.kda_prologue(*xs_t, *ws_t, H, out_dtype=torch.float32)
    q1, k1, v1, st1 = axiom_amd.kda_prologue(*(x[:, :17].contiguous() for x in xs_t), *ws_t, H,
                                             out_dtype=torch.float32)
    # second segment updates the buffers in place (b*_in == b*_out at the C ABI)
    L = axiom_amd._lib.lib()
    from axiom_amd.kda import _ptr, _stream
    x2 = [x[:, 17:].contiguous() for x in xs_t]
    q2, k2, v2 = (torch.empty((B, T - 17, H, d), device=cuda) for _ in range(3))
    rc = L.kda_prologue(_stream(cuda), *(_ptr(x) for x in x2), *(_ptr(w) for w in ws_t),
                        *(_ptr(b) for b in st1), *(_ptr(b) for b in st1), _ptr(q2), _ptr(k2), _ptr(v2),
                        B, T - 17, H, d, K, 0, 0)
    assert rc == 0, axiom_amd._lib.last_error()
    torch.cuda.synchronize()
    assert torch.equal(torch.cat([q1, q2], 1), q) and torch.equal(torch.cat([v1, v2], 1), v)
    for a, b in zip(st1, st):
        assert torch.equal(a, b)


@pytest.mark.parametrize("o_dt,g_dt,y_dt,dv", [
    (torch.float32, torch.float32, torch.float32, 128),
    (torch.float32, torch.bfloat16, torch.bfloat16, 128),
    (torch.bfloat16, torch.float32, torch.float32, 64),
])
def test_epilogue_matches_oracle(cuda, o_dt, g_dt, y_dt, dv):
    import axiom_amd
    rng = np.random.default_rng(dv)
    B, T, H = 2, 33, 3
    o = rng.standard_normal((B, T, H, dv)).astype(np.float32)
    o[0, 0, 0] = 0.0                                   # an all-zero head row: output 0, not NaN
    gate = rng.standard_normal((B, T, H * dv)).astype(np.float32)
    y = axiom_amd.kda_epilogue(torch.from_numpy(o).to(cuda, o_dt), torch.from_numpy(gate).to(cuda, g_dt),
                               eps=1e-6, out_dtype=y_dt)
    torch.cuda.synchronize()
    ref = Lr.epilogue(_as(o, o_dt), _as(gate, g_dt), eps=1e-6)
    _close(y, ref, o_dt == g_dt == y_dt == torch.float32)


@pytest.mark.parametrize("dt,d,Kc", [(torch.float32, 128, 4), (torch.bfloat16, 64, 4), (torch.float32, 64, 1),
                                     (torch.bfloat16, 128, 8), (torch.float32, 128, 2)])
def test_decode_layer_steps_equal_the_whole_sequence(cuda, dt, d, Kc):
    """T layer steps (conv buffers and state carried in place) == prologue over the
    T tokens, the recurrence, and the epilogue (the decode == chunked invariant of
    the reference's generation path, net/kda.py:277-295)."""
    import axiom_amd
    from oracle import inputs, kda_oracle as K
    B, T, H = 2, 12, 2
    rng = np.random.default_rng(d + Kc)
    xs, ws, _ = _proj(B, T, H, d, Kc, seed=d + 1)
    base = inputs.make_inputs(B, T, H, d, d, seed=d + 2, dtype="fp32")
    gate = rng.standard_normal((B, T, H * d)).astype(np.float32)
    S0 = (rng.standard_normal((B, H, d, d)) * 0.05).astype(np.float32)
    xs_r = [_as(x, dt) for x in xs]
    g_r, b_r, gate_r = _as(base["g"], dt), _as(base["beta"], dt), _as(gate, dt)
    q, k, v, _ = Lr.prologue(*xs_r, *ws, H)
    if dt == torch.bfloat16:   # the layer step hands bf16 q, k, v to the decode kernel
        q, k, v = (_as(x.astype(np.float32), dt) for x in (q, k, v))
    o, hT = K.recurrent_fwd(q, k, v, g_r, b_r, h0=S0)
    y_ref = Lr.epilogue(o, gate_r)
    state = torch.from_numpy(S0).to(cuda)
    bufs = tuple(torch.zeros((B, Kc - 1, H * d), device=cuda) for _ in range(3))
    ws_t = [torch.from_numpy(w).to(cuda) for w in ws]
    ys = []
    for t in range(T):
        args = [torch.from_numpy(np.ascontiguousarray(x[:, t])).to(cuda, dt) for x in xs]
        g_t = torch.from_numpy(np.ascontiguousarray(base["g"][:, t])).to(cuda, dt)
        b_t = torch.from_numpy(np.ascontiguousarray(base["beta"][:, t])).to(cuda, dt)
        gt_t = torch.from_numpy(np.ascontiguousarray(gate[:, t])).to(cuda, dt)
        ys.append(axiom_amd.kda_decode_layer_step(*args, g_t, b_t, gt_t, *ws_t, bufs, state))
    torch.cuda.synchronize()
    y = torch.stack(ys, 1).double().cpu().numpy()
    if dt == torch.float32:
        assert np.abs(y - y_ref).max() <= 1e-4, np.abs(y - y_ref).max()
        assert np.abs(state.cpu().numpy() - hT).max() <= 1e-5
    else:
        assert np.linalg.norm(y - y_ref) / np.linalg.norm(y_ref) <= 1e-2
        assert np.linalg.norm(state.cpu().numpy() - hT) / np.linalg.norm(hT) <= 1e-2
    for buf, x in zip(bufs, xs_r):
        np.testing.assert_allclose(buf.cpu().numpy(), x[:, T - (Kc - 1):] if Kc > 1 else x[:, :0],
                                   rtol=0, atol=0)
