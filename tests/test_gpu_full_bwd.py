"""GPU parity of the backward at the benchmarked shape and with many chains.

The chunked backward (kda_chunk_bwd) and the layer backward (kda_layer's
autograd) run whole at config 1 (B4 T4096 H16 d128, bf16 inputs); sampled
(batch, head) chains are compared with the float64 oracle over their full
length (chains are independent, so a sample is exact for its chains).  The
sample covers every batch row of the heads it takes, so the conv-tap
gradients (summed over the batch) of those heads' channels are checked too.
A small case with B*H = 12 chains exercises the scans' chain -> workgroup
mapping beyond the first XCD slot.  Bars as tests/test_gpu_bwd.py (chunked,
16-bit inputs: relative L2 <= 1e-3, max-abs <= 2e-3 x max|ref| against the
float64 oracle) and tests/test_gpu_layer_bwd.py (layer with bf16
projections: 1e-2 / 5e-2).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import inputs, kda_oracle as K, layer as Lr
from tests.kda_testutil import make_inputs_device

pytestmark = pytest.mark.gpu

NAMES = ("dq", "dk", "dv", "dg", "dbeta", "dh0")
REL16, ABS16 = 1e-3, 2e-3   # chunked backward, 16-bit inputs (tests/test_gpu_bwd.py)


def _close(name, got, ref, rel_tol, abs_tol):
    got = got.double().cpu().numpy() if isinstance(got, torch.Tensor) else np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    assert np.all(np.isfinite(got)), f"{name}: non-finite"
    rel = K.rel_l2(got, ref)
    mx = K.max_abs(got, ref)
    scale = max(1.0, float(np.abs(ref).max()))
    print(f"{name}: rel_l2={rel:.2e} max_abs={mx:.2e}", flush=True)
    assert rel <= rel_tol and mx <= abs_tol * scale, f"{name}: rel_l2={rel:.3e} max_abs={mx:.3e}"


@pytest.mark.parametrize("d", [64, 128])
def test_bwd_many_chains(cuda, d):
    """B=3, H=4: twelve chains, so the scans' workgroups of chains 8..11 (the
    second slot of each XCD) are checked as well as the first eight."""
    import axiom_amd
    B, T, H = 3, 200, 4
    x = inputs.make_inputs(B, T, H, d, d, seed=31 + d, dtype="bf16", h0_std=0.05)
    rng = np.random.default_rng(32 + d)
    do = rng.standard_normal((B, T, H, d)).astype(np.float32)
    dht = (rng.standard_normal((B, H, d, d)) * 0.1).astype(np.float32)
    t = {n: torch.from_numpy(x[n]).to(cuda, torch.bfloat16) for n in ("q", "k", "v", "g", "beta")}
    out = axiom_amd.kda_chunk_bwd(t["q"], t["k"], t["v"], t["g"], t["beta"], torch.from_numpy(do).to(cuda),
                                  dht=torch.from_numpy(dht).to(cuda),
                                  initial_state=torch.from_numpy(x["h0"]).to(cuda))
    torch.cuda.synchronize()
    ref = K.chunk_bwd(x["q"], x["k"], x["v"], x["g"], x["beta"], do.astype(np.float64),
                      dht=dht.astype(np.float64), h0=x["h0"], chunk=64)
    for n, got, r in zip(NAMES, out, ref):
        _close(n, got, r, REL16, ABS16)


def test_bwd_config1_full(cuda):
    import axiom_amd
    B, T, H, d = 4, 4096, 16, 128
    x = make_inputs_device(B, T, H, d, d, seed=111, device=cuda)
    gen = torch.Generator(device=cuda)
    gen.manual_seed(112)
    do = torch.randn(B, T, H, d, device=cuda, generator=gen)
    dht = torch.randn(B, H, d, d, device=cuda, generator=gen) * 0.1
    print("[full] config 1 backward", flush=True)
    out = axiom_amd.kda_chunk_bwd(x["q"], x["k"], x["v"], x["g"], x["beta"], do, dht=dht)
    torch.cuda.synchronize()
    for t in out:
        assert torch.isfinite(t).all()
    heads = [0, 7, 15]
    hc = {n: x[n][:, :, heads].float().cpu().numpy() for n in ("q", "k", "v", "g", "beta")}
    ref = K.chunk_bwd(hc["q"], hc["k"], hc["v"], hc["g"], hc["beta"],
                      do[:, :, heads].double().cpu().numpy(),
                      dht=dht[:, heads].double().cpu().numpy(), chunk=64)
    for n, got, r in zip(NAMES, out, ref):
        sub = got[:, heads] if n == "dh0" else got[:, :, heads]
        _close(n, sub, r, REL16, ABS16)


def test_layer_bwd_config1_full(cuda):
    """kda_layer forward + backward at B4 T4096 H16 d128 K4 with bf16
    projections, gate and output; heads 0 and 15 of every batch row against
    the oracle's chain (prologue -> chunk_fwd -> epilogue_bwd -> chunk_bwd ->
    prologue_bwd), conv taps and carried buffers included."""
    import axiom_amd
    B, T, H, d, K_ = 4, 4096, 16, 128, 4
    HD = H * d
    gen = torch.Generator(device=cuda)
    gen.manual_seed(121)
    bf = torch.bfloat16

    def rnd(*shape, s=1.0, dt=torch.float32):
        return (torch.randn(*shape, device=cuda, generator=gen) * s).to(dt)

    xs = [rnd(B, T, HD, dt=bf) for _ in range(3)]
    ws = [rnd(K_, HD, s=0.4) for _ in range(3)]
    bufs = [rnd(B, K_ - 1, HD) for _ in range(3)]
    z = rnd(B, T, HD, dt=bf)
    gz = torch.randn(B, T, H, d, device=cuda, generator=gen)
    a = torch.rand(H, device=cuda, generator=gen) * -2.0
    g = (-torch.nn.functional.softplus(gz) * torch.exp(a)[None, None, :, None]).to(bf)
    beta = torch.sigmoid(torch.randn(B, T, H, device=cuda, generator=gen)).to(bf)
    h0 = rnd(B, H, d, d, s=0.02)
    dy = rnd(B, T, HD, dt=bf)
    dht = rnd(B, H, d, d, s=0.1)
    scale = d ** -0.5
    leaves = [t.clone().requires_grad_(True) for t in (*xs, g, beta, z, *ws, *bufs, h0)]
    xq, xk, xv, gl, bl, zl, wq, wk, wv, bq, bk, bvb, h0l = leaves
    print("[full] config 1 layer forward + backward", flush=True)
    y, ht = axiom_amd.kda_layer(xq, xk, xv, gl, bl, zl, wq, wk, wv, conv_state=(bq, bk, bvb),
                                initial_state=h0l, scale=scale, eps=1e-6)
    ((y.float() * dy.float()).sum() + (ht * dht).sum()).backward()
    torch.cuda.synchronize()

    heads = [0, 15]
    ch = np.concatenate([np.arange(h * d, (h + 1) * d) for h in heads])
    chd = torch.from_numpy(ch).to(cuda)

    def host(t, chan_axis=-1):
        return t.index_select(chan_axis, chd).double().cpu().numpy()

    Hs = len(heads)
    xr = [host(t) for t in xs]
    wr = [host(t) for t in ws]
    br = [host(t) for t in bufs]
    q, k, v, _ = Lr.prologue(*xr, *wr, Hs, bufs=br)
    gr = g[:, :, heads].double().cpu().numpy()
    betar = beta[:, :, heads].double().cpu().numpy()
    h0r = h0[:, heads].double().cpu().numpy()
    o, _ = K.chunk_fwd(q, k, v, gr, betar, h0=h0r, scale=scale)
    do, dz = Lr.epilogue_bwd(o.numpy(), host(z), host(dy), eps=1e-6)
    dq, dk, dv, dg, dbeta, dh0 = K.chunk_bwd(q, k, v, gr, betar, do, dht=dht[:, heads].double().cpu().numpy(),
                                             h0=h0r, scale=scale)
    dqp, dkp, dvp, dw, db = Lr.prologue_bwd(*xr, *wr, Hs, dq, dk, dv, bufs=br)
    checks = [("dqp", xq.grad, dqp, -1), ("dkp", xk.grad, dkp, -1), ("dvp", xv.grad, dvp, -1),
              ("dgate", zl.grad, dz, -1), ("dwq", wq.grad, dw[0], -1), ("dwk", wk.grad, dw[1], -1),
              ("dwv", wv.grad, dw[2], -1), ("dbq", bq.grad, db[0], -1), ("dbk", bk.grad, db[1], -1),
              ("dbv", bvb.grad, db[2], -1)]
    for name, got, r, ax in checks:
        _close(name, host(got, ax), r, 1e-2, 5e-2)
    _close("dg", gl.grad[:, :, heads], dg, 1e-2, 5e-2)
    _close("dbeta", bl.grad[:, :, heads], dbeta, 1e-2, 5e-2)
    _close("dh0", h0l.grad[:, heads], dh0, 1e-2, 5e-2)
