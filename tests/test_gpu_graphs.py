"""The entry points inside HIP graphs (torch.cuda.CUDAGraph on ROCm).

No compute entry point allocates, synchronises or sets memory with
hipMemsetAsync, so a caller can capture them on its stream: the chunked
forward, a run of layer decode steps, and the layer's backward chain.  Each test
captures a sequence of calls, replays the graph several times with the
program's own eager work and synchronisations between the replays, and checks
every replay against the eager result bit for bit.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import inputs
from tests.kda_testutil import to_dev

pytestmark = pytest.mark.gpu


def _capture(fn):
    """Warm up on a side stream, then capture fn() into a graph."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn()
    torch.cuda.synchronize()
    return g, out


def test_chunk_fwd_graph_replays_match_eager(cuda):
    import axiom_amd
    from axiom_amd import kda as kmod
    d = inputs.make_inputs(2, 200, 4, 128, 128, seed=41, dtype="bf16", h0_std=0.05)
    q, k, v, g, beta = (to_dev(d[n], torch.bfloat16, cuda) for n in ("q", "k", "v", "g", "beta"))
    h0 = to_dev(d["h0"], torch.float32, cuda)
    ws = torch.empty(kmod.chunk_fwd_workspace_bytes(2, 200, 4, 128, 128), dtype=torch.uint8, device=cuda)
    o_ref, ht_ref = axiom_amd.kda_chunk_fwd(q, k, v, g, beta, initial_state=h0, workspace=ws)
    torch.cuda.synchronize()
    graph, (o, ht) = _capture(lambda: axiom_amd.kda_chunk_fwd(q, k, v, g, beta, initial_state=h0, workspace=ws))
    for rep in range(3):
        o.zero_()
        ht.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(o, o_ref) and torch.equal(ht, ht_ref), f"replay {rep}"
        # eager work between replays on the same buffers the graph reads
        axiom_amd.kda_chunk_fwd(q, k, v, g, beta, initial_state=h0, workspace=ws)
        torch.cuda.synchronize()


def test_decode_layer_steps_graph_replays_match_eager(cuda):
    """Eight layer decode steps (conv buffers and state carried in place) in one graph."""
    import axiom_amd
    B, H, d, K, steps = 2, 4, 64, 4, 8
    rng = np.random.default_rng(42)
    dt = torch.bfloat16
    toks = [[to_dev(rng.standard_normal((B, H * d)).astype(np.float32), dt, cuda) for _ in range(3)]
            for _ in range(steps)]
    base = inputs.make_inputs(steps, B, H, d, d, seed=43, dtype="bf16")
    gs = [to_dev(base["g"][t], dt, cuda) for t in range(steps)]
    bs = [to_dev(base["beta"][t], dt, cuda) for t in range(steps)]
    gates = [to_dev(rng.standard_normal((B, H * d)).astype(np.float32), dt, cuda) for _ in range(steps)]
    ws_ = [to_dev((rng.standard_normal((K, H * d)) * 0.4).astype(np.float32), torch.float32, cuda)
           for _ in range(3)]
    S0 = to_dev((rng.standard_normal((B, H, d, d)) * 0.05).astype(np.float32), torch.float32, cuda)
    bufs0 = [to_dev(rng.standard_normal((B, K - 1, H * d)).astype(np.float32), torch.float32, cuda)
             for _ in range(3)]
    state = S0.clone()
    bufs = [b.clone() for b in bufs0]

    def run():
        return [axiom_amd.kda_decode_layer_step(*toks[t], gs[t], bs[t], gates[t], *ws_, bufs, state)
                for t in range(steps)]

    ys_ref = [y.clone() for y in run()]
    state_ref, bufs_ref = state.clone(), [b.clone() for b in bufs]
    graph, ys = None, None
    state.copy_(S0)
    for b, b0 in zip(bufs, bufs0):
        b.copy_(b0)
    graph, ys = _capture(run)   # the warm-up inside advanced the state: reset before each replay
    for rep in range(3):
        state.copy_(S0)
        for b, b0 in zip(bufs, bufs0):
            b.copy_(b0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for t in range(steps):
            assert torch.equal(ys[t], ys_ref[t]), f"replay {rep} token {t}"
        assert torch.equal(state, state_ref), f"replay {rep} state"
        for b, br in zip(bufs, bufs_ref):
            assert torch.equal(b, br), f"replay {rep} conv buffer"
        _ = (state * 2.0).sum().item()   # the program's own eager work between replays


def test_layer_backward_chain_graph_replays_match_eager(cuda):
    """kda_epilogue_bwd -> kda_chunk_bwd -> kda_prologue_bwd (the layer's
    backward after the recompute) captured in one graph."""
    import axiom_amd
    from axiom_amd import kda as kmod
    B, T, H, d, K = 2, 150, 2, 128, 4
    rng = np.random.default_rng(44)
    bf = torch.bfloat16
    xs = [to_dev(rng.standard_normal((B, T, H * d)).astype(np.float32), bf, cuda) for _ in range(3)]
    ws_ = [to_dev((rng.standard_normal((K, H * d)) * 0.4).astype(np.float32), torch.float32, cuda) for _ in range(3)]
    bufs = tuple(to_dev(rng.standard_normal((B, K - 1, H * d)).astype(np.float32), torch.float32, cuda)
                 for _ in range(3))
    base = inputs.make_inputs(B, T, H, d, d, seed=45, dtype="bf16")
    g, beta = to_dev(base["g"], bf, cuda), to_dev(base["beta"], bf, cuda)
    gate = to_dev(rng.standard_normal((B, T, H * d)).astype(np.float32), bf, cuda)
    dy = to_dev(rng.standard_normal((B, T, H * d)).astype(np.float32), bf, cuda)
    q, k, v, _ = axiom_amd.kda_prologue(*xs, *ws_, H, conv_state=bufs, return_state=False)
    o, _ = axiom_amd.kda_chunk_fwd(q, k, v, g, beta, output_final_state=False)
    bws = torch.empty(kmod.chunk_bwd_workspace_bytes(B, T, H, d, d), dtype=torch.uint8, device=cuda)
    pws = torch.empty(kmod.prologue_bwd_workspace_bytes(B, T, H, d, K), dtype=torch.uint8, device=cuda)

    def run():
        do, dgate = axiom_amd.kda_epilogue_bwd(o, gate, dy)
        dq, dk, dv, dg, dbeta, _ = axiom_amd.kda_chunk_bwd(q, k, v, g, beta, do, need_dh0=False, workspace=bws)
        dx, dw, db = axiom_amd.kda_prologue_bwd(*xs, *ws_, dq, dk, dv, conv_state=bufs, workspace=pws)
        return [dgate, dg, dbeta, *dx, *dw, *db]

    ref = [t.clone() for t in run()]
    torch.cuda.synchronize()
    graph, outs = _capture(run)
    for rep in range(3):
        for t in outs:
            t.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for i, (got, want) in enumerate(zip(outs, ref)):
            assert torch.equal(got, want), f"replay {rep} output {i}"
        run()   # eager work on the same workspaces between replays
        torch.cuda.synchronize()


def test_noalloc_captured_first_call_replays_match_eager(cuda):
    """kda_chunk_fwd_noalloc captured into a graph with no warm-up call, so its
    first call on the device -- the lookup of the library scratch's device
    address -- happens during the capture (no other test of the suite calls
    it before this one).  Replays, with eager calls of both entry points on
    the same buffers between them, equal the eager kda_chunk_fwd bit for bit;
    a second graph of a smaller call reuses the same scratch."""
    import ctypes
    from axiom_amd import _lib
    L = _lib.lib()
    p = lambda a: ctypes.c_void_p(0 if a is None else a.data_ptr())  # noqa: E731

    def case(B, T, H, seed):
        d = inputs.make_inputs(B, T, H, 128, 128, seed=seed, dtype="bf16", h0_std=0.05)
        t = {n: to_dev(d[n], torch.bfloat16, cuda) for n in ("q", "k", "v", "g", "beta")}
        t["h0"] = to_dev(d["h0"], torch.float32, cuda)
        t["o"] = torch.zeros(B, T, H, 128, device=cuda)
        t["ht"] = torch.zeros(B, H, 128, 128, device=cuda)
        return t

    def args(t, B, T, H, o, ht):
        stream = ctypes.c_void_p(torch.cuda.current_stream(cuda).cuda_stream)
        return (stream, p(t["q"]), p(t["k"]), p(t["v"]), p(t["g"]), p(t["beta"]), p(t["h0"]), ctypes.c_void_p(0), 0,
                p(o), p(ht), B, T, H, 128, 128, 64, 1.0, _lib.KDA_DTYPE_BF16, _lib.KDA_DTYPE_F32)

    def eager_ref(t, B, T, H):
        o, ht = torch.empty_like(t["o"]), torch.empty_like(t["ht"])
        nb = int(L.kda_chunk_fwd_workspace(B, T, H, 128, 128, 64, 0, _lib.KDA_DTYPE_BF16))
        ws = torch.empty(nb, dtype=torch.uint8, device=cuda)
        assert L.kda_chunk_fwd(*args(t, B, T, H, o, ht), p(ws), nb) == 0, _lib.last_error()
        torch.cuda.synchronize()
        return o, ht

    graphs = []
    for B, T, H, seed in ((2, 1000, 4, 51), (1, 130, 2, 52)):
        t = case(B, T, H, seed)
        g = torch.cuda.CUDAGraph()
        print(f"[graph noalloc] capture B={B} T={T} H={H}", flush=True)
        with torch.cuda.graph(g):
            rc = L.kda_chunk_fwd_noalloc(*args(t, B, T, H, t["o"], t["ht"]))
        torch.cuda.synchronize()
        assert rc == _lib.KDA_OK, _lib.last_error()
        graphs.append((g, t, B, T, H))
    for g, t, B, T, H in graphs:
        o_ref, ht_ref = eager_ref(t, B, T, H)
        for rep in range(3):
            t["o"].zero_()
            t["ht"].zero_()
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(t["o"], o_ref) and torch.equal(t["ht"], ht_ref), f"B={B} T={T} replay {rep}"
            # eager calls between replays, through both entry points
            o2, ht2 = torch.empty_like(o_ref), torch.empty_like(ht_ref)
            assert L.kda_chunk_fwd_noalloc(*args(t, B, T, H, o2, ht2)) == 0, _lib.last_error()
            torch.cuda.synchronize()
            assert torch.equal(o2, o_ref) and torch.equal(ht2, ht_ref)
            eager_ref(t, B, T, H)
