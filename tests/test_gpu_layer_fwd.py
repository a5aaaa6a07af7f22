"""GPU parity of the chunked layer forward (kda_layer_fwd).

The layer is prologue -> chunked scan -> epilogue (net/kda.py:790-853 between
the projections and W_o).  With bf16 projections and K <= 4 taps the prologue
runs inside the intra kernel; that fused path is checked bit for bit against
the three standalone entry points (kda_prologue -> kda_chunk_fwd ->
kda_epilogue, each pinned against the oracle in its own tests), at small
shapes and at the full config-1 shape (three T-segments).  The layer as a whole
is checked against the float64 oracle chain (oracle/layer.py prologue, q, k, v
rounded to bf16 as the layer hands them to the scan, kda_oracle.chunk_fwd,
epilogue): bf16 projections rel-L2 <= 2e-3 and max-abs <= 2e-2 on y (fp32 out),
the bf16 bar of the scan itself; fp32 projections max-abs <= 1e-4.  Calls
chained through the conv buffers and the state equal one call over the whole
sequence (bit for bit when the first call ends on a chunk boundary).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import inputs, kda_oracle as Ko, layer as Lr

pytestmark = pytest.mark.gpu


def _as(x, dt):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dt).double().numpy()


def _dev(cuda, x, dt):
    return torch.from_numpy(np.ascontiguousarray(x)).to(cuda, dt)


def _case(B, T, H, d, Kc, seed, bufs=True, h0=True):
    rng = np.random.default_rng(seed)
    xs = [rng.standard_normal((B, T, H * d)).astype(np.float32) for _ in range(3)]
    ws = [(rng.standard_normal((Kc, H * d)) * 0.4).astype(np.float32) for _ in range(3)]
    bs = [rng.standard_normal((B, Kc - 1, H * d)).astype(np.float32) for _ in range(3)] if bufs else None
    base = inputs.make_inputs(B, T, H, d, d, seed=seed + 1, dtype="fp32")
    gate = rng.standard_normal((B, T, H * d)).astype(np.float32)
    S0 = (rng.standard_normal((B, H, d, d)) * 0.05).astype(np.float32) if h0 else None
    return dict(xs=xs, ws=ws, bs=bs, g=base["g"], beta=base["beta"], gate=gate, S0=S0, H=H)


def _tensors(cuda, c, dt, gdt):
    xs = [_dev(cuda, x, dt) for x in c["xs"]]
    ws = [_dev(cuda, w, torch.float32) for w in c["ws"]]
    bs = None if c["bs"] is None else tuple(_dev(cuda, b, torch.float32) for b in c["bs"])
    S0 = None if c["S0"] is None else _dev(cuda, c["S0"], torch.float32)
    return xs, ws, bs, _dev(cuda, c["g"], gdt), _dev(cuda, c["beta"], gdt), _dev(cuda, c["gate"], dt), S0


def _layer(cuda, c, dt, gdt, out_dtype=torch.float32, with_o=False):
    import axiom_amd
    xs, ws, bs, g, beta, gate, S0 = _tensors(cuda, c, dt, gdt)
    o = torch.full(g.shape, float("nan"), device=cuda) if with_o else None
    y, ht, new = axiom_amd.kda_layer_fwd(*xs, g, beta, gate, *ws, conv_state=bs, initial_state=S0,
                                         out_dtype=out_dtype, o_out=o)
    torch.cuda.synchronize()
    return (y, ht, new, o) if with_o else (y, ht, new)


def _unfused(cuda, c, dt, gdt, out_dtype=torch.float32, with_o=False):
    import axiom_amd
    xs, ws, bs, g, beta, gate, S0 = _tensors(cuda, c, dt, gdt)
    q, k, v, new = axiom_amd.kda_prologue(*xs, *ws, c["H"], conv_state=bs, out_dtype=dt)
    o, ht = axiom_amd.kda_chunk_fwd(q, k, v, g, beta, initial_state=S0)
    y = axiom_amd.kda_epilogue(o, gate, eps=1e-6, out_dtype=out_dtype)
    torch.cuda.synchronize()
    return (y, ht, new, o) if with_o else (y, ht, new)


def _oracle(c, dt, gdt):
    xs_r = [_as(x, dt) for x in c["xs"]]
    q, k, v, new = Lr.prologue(*xs_r, *c["ws"], c["H"], bufs=c["bs"])
    if dt == torch.bfloat16:      # the layer hands bf16 q, k, v to the scan
        q, k, v = (_as(x.astype(np.float32), dt) for x in (q, k, v))
    o, hT = Ko.chunk_fwd(q, k, v, _as(c["g"], gdt), _as(c["beta"], gdt), h0=c["S0"])
    y = Lr.epilogue(o.numpy(), _as(c["gate"], dt), eps=1e-6)
    return y, hT.numpy(), new


@pytest.mark.parametrize("B,T,H,d,Kc,gdt,bufs,h0", [
    (2, 200, 2, 128, 4, torch.bfloat16, True, True),
    (1, 64, 3, 64, 4, torch.bfloat16, True, False),
    (1, 130, 2, 128, 3, torch.float32, False, True),     # bf16 projections, fp32 gates
    (2, 37, 2, 64, 2, torch.bfloat16, True, True),
    (1, 1, 2, 128, 4, torch.bfloat16, True, True),       # one token
    (2, 3, 2, 64, 4, torch.bfloat16, True, False),       # T < K - 1
    (1, 129, 1, 128, 1, torch.bfloat16, False, False),   # K = 1: no history
])
def test_fused_layer_equals_the_three_entry_points(cuda, B, T, H, d, Kc, gdt, bufs, h0):
    c = _case(B, T, H, d, Kc, seed=T + d + Kc, bufs=bufs, h0=h0)
    print(f"[layer fused vs unfused] B={B} T={T} H={H} d={d} K={Kc} gates={gdt}", flush=True)
    y, ht, new, o = _layer(cuda, c, torch.bfloat16, gdt, with_o=True)
    y2, ht2, new2, o2 = _unfused(cuda, c, torch.bfloat16, gdt, with_o=True)
    assert torch.equal(y, y2), (y - y2).abs().max().item()
    assert torch.equal(ht, ht2)
    assert torch.equal(o, o2)          # o_out: the scan's output, as kda_chunk_fwd's
    for a, b in zip(new, new2):
        assert torch.equal(a, b)


@pytest.mark.parametrize("B,T,H,d,Kc,dt,gdt", [
    (2, 150, 2, 128, 4, torch.bfloat16, torch.bfloat16),
    (1, 100, 2, 64, 4, torch.bfloat16, torch.float32),
    (1, 90, 2, 128, 6, torch.bfloat16, torch.bfloat16),   # K > 4: prologue as its own pass
    (2, 70, 2, 64, 4, torch.float32, torch.float32),      # fp32: exact kernels
])
def test_layer_matches_oracle(cuda, B, T, H, d, Kc, dt, gdt):
    c = _case(B, T, H, d, Kc, seed=3 * T + d)
    print(f"[layer vs oracle] B={B} T={T} H={H} d={d} K={Kc} {dt} gates={gdt}", flush=True)
    y, ht, new = _layer(cuda, c, dt, gdt)
    y_ref, hT_ref, new_ref = _oracle(c, dt, gdt)
    y = y.double().cpu().numpy()
    ht = ht.double().cpu().numpy()
    if dt == torch.float32:
        assert np.abs(y - y_ref).max() <= 1e-4, np.abs(y - y_ref).max()
        assert np.abs(ht - hT_ref).max() <= 1e-5
    else:
        assert Ko.rel_l2(y, y_ref) <= 2e-3 and Ko.max_abs(y, y_ref) <= 2e-2, (Ko.rel_l2(y, y_ref), Ko.max_abs(y, y_ref))
        assert Ko.rel_l2(ht, hT_ref) <= 1e-3
    for a, b in zip(new, new_ref):
        np.testing.assert_array_equal(a.double().cpu().numpy(), b)


def test_layer_calls_chain_through_conv_buffers_and_state(cuda):
    """Two calls (the first ending on a chunk boundary) == one call, bit for bit."""
    import axiom_amd
    B, T1, T2, H, d, Kc = 2, 128, 100, 2, 128, 4
    c = _case(B, T1 + T2, H, d, Kc, seed=11)
    xs, ws, bs, g, beta, gate, S0 = _tensors(cuda, c, torch.bfloat16, torch.bfloat16)
    y, ht, new = axiom_amd.kda_layer_fwd(*xs, g, beta, gate, *ws, conv_state=bs, initial_state=S0,
                                         out_dtype=torch.float32)
    sl = lambda t, a, b: t[:, a:b].contiguous()  # noqa: E731
    y1, h1, n1 = axiom_amd.kda_layer_fwd(*(sl(x, 0, T1) for x in xs), sl(g, 0, T1), sl(beta, 0, T1),
                                         sl(gate, 0, T1), *ws, conv_state=bs, initial_state=S0,
                                         out_dtype=torch.float32)
    y2, h2, n2 = axiom_amd.kda_layer_fwd(*(sl(x, T1, T1 + T2) for x in xs), sl(g, T1, T1 + T2),
                                         sl(beta, T1, T1 + T2), sl(gate, T1, T1 + T2), *ws, conv_state=n1,
                                         initial_state=h1, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(torch.cat([y1, y2], 1), y)
    assert torch.equal(h2, ht)
    for a, b in zip(n2, new):
        assert torch.equal(a, b)


def test_fused_layer_equals_the_three_entry_points_at_config1(cuda):
    """B=4 T=4096 H=16 d=128 (three T-segments of the scan), K=4, bf16."""
    import axiom_amd
    B, T, H, d, Kc = 4, 4096, 16, 128, 4
    gen = torch.Generator(device=cuda)
    gen.manual_seed(7)
    xs = [torch.randn(B, T, H * d, device=cuda, generator=gen).to(torch.bfloat16) for _ in range(3)]
    ws = [torch.randn(Kc, H * d, device=cuda, generator=gen) * 0.4 for _ in range(3)]
    g = (-torch.nn.functional.softplus(torch.randn(B, T, H, d, device=cuda, generator=gen))).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn(B, T, H, device=cuda, generator=gen)).to(torch.bfloat16)
    gate = torch.randn(B, T, H * d, device=cuda, generator=gen).to(torch.bfloat16)
    y, ht, _ = axiom_amd.kda_layer_fwd(*xs, g, beta, gate, *ws, out_dtype=torch.bfloat16, return_conv_state=False)
    q, k, v, _ = axiom_amd.kda_prologue(*xs, *ws, H, out_dtype=torch.bfloat16, return_state=False)
    o, ht2 = axiom_amd.kda_chunk_fwd(q, k, v, g, beta)
    y2 = axiom_amd.kda_epilogue(o, gate, eps=1e-6, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.isfinite(y.float()).all()
    assert torch.equal(y, y2) and torch.equal(ht, ht2)


@pytest.mark.parametrize("d,gdt", [(128, torch.bfloat16), (64, torch.bfloat16), (128, torch.float32)])
def test_fused_layer_decay_spikes(cuda, d, gdt):
    """Single steps that decay by e^-150 in 3 % of the gate entries put some
    16-row tiles past 2^-100, where the intra kernel takes its anchored path
    and re-reads q and k per level.  With the fused prologue those are the
    convolved, normalised rows, which exist only inside the kernel: the
    fused layer must equal the three entry points (whose scan reads the
    prologue's q, k from memory) bit for bit, and the oracle chain with the
    token-by-token recurrence (the chunked oracle leaves float64's range
    under such decay)."""
    B, T, H, Kc = 2, 192, 2, 4
    c = _case(B, T, H, d, Kc, seed=17 + d)
    rng = np.random.default_rng(23 + d)
    c["g"] = np.where(rng.random(c["g"].shape) < 0.03, np.float32(-150.0), c["g"]).astype(np.float32)
    assert (c["g"].reshape(B, T // 16, 16, H, d).sum(axis=2) / np.log(2.0)).min() < -100.0
    print(f"[layer decay spikes] d={d} gates={gdt}", flush=True)
    y, ht, new, o = _layer(cuda, c, torch.bfloat16, gdt, with_o=True)
    y2, ht2, new2, o2 = _unfused(cuda, c, torch.bfloat16, gdt, with_o=True)
    assert torch.isfinite(y).all() and torch.isfinite(ht).all()
    assert torch.equal(o, o2), (o - o2).abs().max().item()
    assert torch.equal(y, y2) and torch.equal(ht, ht2)
    xs_r = [_as(x, torch.bfloat16) for x in c["xs"]]
    q, k, v, _ = Lr.prologue(*xs_r, *c["ws"], c["H"], bufs=c["bs"])
    q, k, v = (_as(x.astype(np.float32), torch.bfloat16) for x in (q, k, v))
    o_ref, hT_ref = Ko.recurrent_fwd(q, k, v, _as(c["g"], gdt), _as(c["beta"], gdt), h0=c["S0"])
    o_ref, hT_ref = np.asarray(o_ref), np.asarray(hT_ref)
    y_ref = Lr.epilogue(o_ref, _as(c["gate"], torch.bfloat16), eps=1e-6)
    o_np = o.double().cpu().numpy()
    assert Ko.rel_l2(o_np, o_ref) <= 1e-3 and Ko.max_abs(o_np, o_ref) <= 2e-2, (Ko.rel_l2(o_np, o_ref), Ko.max_abs(o_np, o_ref))
    y_np = y.double().cpu().numpy()
    assert Ko.rel_l2(y_np, y_ref) <= 2e-3 and Ko.max_abs(y_np, y_ref) <= 2e-2, (Ko.rel_l2(y_np, y_ref), Ko.max_abs(y_np, y_ref))
    ht_np = ht.double().cpu().numpy()
    assert Ko.rel_l2(ht_np, hT_ref) <= 1e-3
