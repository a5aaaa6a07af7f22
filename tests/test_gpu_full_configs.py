"""GPU parity at the full sizes of the benchmark configurations.

Each test combines
* the fp64 oracle on every chain (every (sequence, head) pair, at its full
  length; the oracle runs these sizes in seconds on the host's threads), each
  chain held to the bar on its own so that one wrong chain -- a slip in the
  chain -> workgroup or XCD mapping, the longest-first varlen order, a
  segment boundary -- cannot hide in a norm over all of them, and
* size-independent properties: splitting a sequence and carrying the final
  state across gives the same result bit for bit; a packed varlen run equals
  the per-sequence runs bit for bit; no non-finite values.

Config 1: B4 T4096 H16 d128; config 2: B1 T65536 H16 d128 (1024 serial
chunks per chain); config 3: 64 sequences of U[128, 8192] tokens packed with
cu_seqlens, H16 d128, per-sequence h0 ~ N(0, 0.02^2); config 4: decode B256
H16 d128 with the fp32 state updated in place for 128 steps.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import inputs, kda_oracle as K
from tests.kda_testutil import (TOL, assert_chain_errors, assert_chains_close, assert_close, chain_errors,
                                host_chains, make_inputs_device)

pytestmark = pytest.mark.gpu


def _fwd(d, h0=None, cu=None):
    import axiom_amd
    o, ht = axiom_amd.kda_chunk_fwd(d["q"], d["k"], d["v"], d["g"], d["beta"], initial_state=h0,
                                    cu_seqlens=cu)
    torch.cuda.synchronize()
    return o, ht


def _slice(d, t0, t1):
    return {n: d[n][:, t0:t1].contiguous() for n in ("q", "k", "v", "g", "beta")}


def _host(d):
    """float32 host copies of the whole inputs (the bf16 values exactly)."""
    return {n: d[n].float().cpu().numpy() for n in ("q", "k", "v", "g", "beta")}


def _all_chains_dense(name, d, o, ht, h0=None):
    """Every (batch row, head) chain against the fp64 oracle, each on its own."""
    x = _host(d)
    o_ref, ht_ref = K.chunk_fwd(x["q"], x["k"], x["v"], x["g"], x["beta"], chunk=64,
                                h0=None if h0 is None else h0.cpu().numpy())
    assert_chains_close(f"{name} o", o, o_ref, TOL["bf16"], chain_axes=(0, 2))
    assert_chains_close(f"{name} ht", ht, ht_ref, TOL["bf16"], chain_axes=(0, 1))


def test_config1_full(cuda):
    B, T, H, dd = 4, 4096, 16, 128
    d = make_inputs_device(B, T, H, dd, dd, seed=101, device=cuda)
    print("[full] config 1 forward", flush=True)
    o, ht = _fwd(d)
    assert torch.isfinite(o).all() and torch.isfinite(ht).all()
    _all_chains_dense("config 1", d, o, ht)
    # The whole call runs in segments of chunks (its intra-chunk results
    # exceed the per-segment budget); four calls of 16 chunks each carry the
    # state between them: same result bit for bit.
    h, outs = None, []
    for t0 in range(0, T, 1024):
        oi, h = _fwd(_slice(d, t0, t0 + 1024), h0=h)
        outs.append(oi)
    assert torch.equal(torch.cat(outs, dim=1), o) and torch.equal(h, ht)
    # Without a final-state output the segments carry the state through the
    # workspace instead of ht: o is the same bit for bit.
    import axiom_amd
    o_nf, ht_nf = axiom_amd.kda_chunk_fwd(d["q"], d["k"], d["v"], d["g"], d["beta"], output_final_state=False)
    torch.cuda.synchronize()
    assert ht_nf is None and torch.equal(o_nf, o)


def test_config2_full(cuda):
    B, T, H, dd = 1, 65536, 16, 128
    d = make_inputs_device(B, T, H, dd, dd, seed=102, device=cuda)
    print("[full] config 2 forward", flush=True)
    o, ht = _fwd(d)
    assert torch.isfinite(o).all() and torch.isfinite(ht).all()
    _all_chains_dense("config 2", d, o, ht)
    # state carry: [0, T/2) then [T/2, T) from its final state == the whole run
    half = T // 2
    o1, ht1 = _fwd(_slice(d, 0, half))
    o2, ht2 = _fwd(_slice(d, half, T), h0=ht1)
    assert torch.equal(o1, o[:, :half]) and torch.equal(o2, o[:, half:])
    assert torch.equal(ht2, ht)


def test_config3_varlen_full(cuda):
    H, dd = 16, 128
    lengths = inputs.make_varlen_lengths(64, 128, 8192, seed=3)
    cu = inputs.cu_seqlens_from_lengths(lengths)
    T = int(cu[-1])
    d = make_inputs_device(1, T, H, dd, dd, seed=103, device=cuda, h0_std=0.02, n_states=len(lengths))
    cu_t = torch.from_numpy(cu).to(cuda)
    print(f"[full] config 3 varlen forward T={T}", flush=True)
    o, ht = _fwd(d, h0=d["h0"], cu=cu_t)
    assert torch.isfinite(o).all() and torch.isfinite(ht).all()
    # the least workspace (segments of 141 units instead of 5.8 GB at once):
    # the same result bit for bit
    import axiom_amd
    from axiom_amd import kda as kmod
    ws = torch.empty(kmod.chunk_fwd_workspace_min_bytes(1, T, H, dd, dd, n_seqs=len(lengths)),
                     dtype=torch.uint8, device=cuda)
    assert ws.numel() < 400 * 10 ** 6
    o_s, ht_s = axiom_amd.kda_chunk_fwd(d["q"], d["k"], d["v"], d["g"], d["beta"], initial_state=d["h0"],
                                        cu_seqlens=cu_t, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(o_s, o) and torch.equal(ht_s, ht)
    del ws, o_s, ht_s
    order = np.argsort(lengths)
    picks = sorted({int(order[0]), int(order[-1]), 0, len(lengths) - 1})
    for i in picks:
        a, b = int(cu[i]), int(cu[i + 1])
        oi, hi = _fwd(_slice(d, a, b), h0=d["h0"][i:i + 1].contiguous())
        assert torch.equal(oi, o[:, a:b]), f"sequence {i}: packed o differs from its own run"
        assert torch.equal(hi[0], ht[i]), f"sequence {i}: packed state differs from its own run"
    # every (sequence, head) chain against the fp64 oracle, each on its own
    x = _host(d)
    o_ref, ht_ref = K.chunk_fwd(x["q"], x["k"], x["v"], x["g"], x["beta"], h0=d["h0"].cpu().numpy(),
                                cu_seqlens=cu, chunk=64)
    o_np, o_ref = o.double().cpu().numpy(), o_ref.numpy()
    rel, mx = np.zeros((len(lengths), H)), np.zeros((len(lengths), H))
    for i in range(len(lengths)):
        a, b = int(cu[i]), int(cu[i + 1])
        rel[i], mx[i] = chain_errors(o_np[:, a:b], o_ref[:, a:b], chain_axes=(2,))
    assert_chain_errors("config 3 o", rel, mx, TOL["bf16"])
    assert_chains_close("config 3 ht", ht, ht_ref, TOL["bf16"], chain_axes=(0, 1))


def test_config4_decode_full(cuda):
    import axiom_amd
    B, H, dd, steps = 256, 16, 128, 128
    d = make_inputs_device(steps, B, H, dd, dd, seed=104, device=cuda)   # [steps, B, H, d]
    gen = torch.Generator(device=cuda)
    gen.manual_seed(105)
    S = torch.randn(B, H, dd, dd, device=cuda, generator=gen) * 0.02
    S0 = S.cpu().numpy()
    print("[full] config 4 decode", flush=True)
    outs = []
    for t in range(steps):
        outs.append(axiom_amd.kda_recurrent_step(d["q"][t], d["k"][t], d["v"][t], d["g"][t], d["beta"][t], S))
    torch.cuda.synchronize()
    assert torch.isfinite(S).all()
    # all 4 096 (b, h) chains over the 128 steps, each on its own
    x = _host(d)
    o_ref, S_ref = K.decode_steps_torch(x["q"], x["k"], x["v"], x["g"], x["beta"], S0)
    assert_chains_close("config 4 o", torch.stack(outs), o_ref, (1e-5, 1e-5), chain_axes=(1, 2))
    assert_chains_close("config 4 S", S, S_ref, (1e-5, 1e-5), chain_axes=(0, 1))


def test_two_segment_minimum_overlapped(cuda):
    """B1 T4096 H16 d128 with h0 (the cc_scan seam's per-element shape): one
    segment's worth of intra results, run as two overlapped segments; two
    every chain against the oracle, the call split at the segment boundary and at
    another point gives the same o and final state bit for bit."""
    from tests.test_capi import dense_segments, overlap_eligible
    B, T, H, dd = 1, 4096, 16, 128
    assert overlap_eligible(B, H, dd, 2) and dense_segments(B, T, H, dd, dd, 2) == (2, 32)
    d = make_inputs_device(B, T, H, dd, dd, seed=111, device=cuda, h0_std=0.02)
    print("[full] two-segment minimum", flush=True)
    o, ht = _fwd(d, h0=d["h0"])
    _all_chains_dense("two-segment minimum", d, o, ht, h0=d["h0"])
    for cut in (2048, 64 * 13):
        o1, h1 = _fwd(_slice(d, 0, cut), h0=d["h0"])
        o2, h2 = _fwd(_slice(d, cut, T), h0=h1)
        assert torch.equal(torch.cat([o1, o2], dim=1), o) and torch.equal(h2, ht), cut


def test_long_two_chain_call_against_oracle(cuda):
    """B1 T50000 H2 d128 with h0: two chains whose intra-chunk results exceed
    one segment (the call runs in segments); both chains against the oracle,
    and the final-state-free call gives the same o bit for bit."""
    import axiom_amd
    B, T, H, dd = 1, 50000, 2, 128
    d = make_inputs_device(B, T, H, dd, dd, seed=106, device=cuda, h0_std=0.02)
    print("[full] long two-chain call", flush=True)
    o, ht = _fwd(d, h0=d["h0"])
    hc = host_chains(d, 0, [0, 1])
    o_ref, ht_ref = K.chunk_fwd(hc["q"], hc["k"], hc["v"], hc["g"], hc["beta"], h0=d["h0"].cpu().numpy(),
                                chunk=64)
    assert_close("o", o, o_ref, TOL["bf16"])
    assert_close("ht", ht, ht_ref, TOL["bf16"])
    o2, _ = axiom_amd.kda_chunk_fwd(d["q"], d["k"], d["v"], d["g"], d["beta"], initial_state=d["h0"],
                                    output_final_state=False)
    torch.cuda.synchronize()
    assert torch.equal(o2, o)


@pytest.mark.parametrize("dd,prec", [(128, "bf16"), (64, "bf16"), (128, "fp16"), (128, "bf16_f32gates")])
def test_overlapped_segments_odd_chunk_heads(cuda, dd, prec):
    """B1 T100000 H3: three chains, few enough that each segment's state scan
    runs in one launch with the next segment's intra work; every segment holds
    an odd number of chunk-heads (the last workgroup's second group idles).
    Every chain against the oracle; the call split in two with the state carried
    across gives the same o and final state bit for bit; bf16 o is the fp32 o
    rounded."""
    import axiom_amd
    from tests.test_capi import dense_segments, overlap_eligible
    B, T, H = 1, 100000, 3
    segments, seg = dense_segments(B, T, H, dd, dd, 2)
    NT = -(-T // 64)
    # some segment after the first (their intra work runs in the overlapped
    # launches) has an odd number of chunk-heads
    assert overlap_eligible(B, H, dd, 2) and segments > 1
    assert any(B * min(seg, NT - i * seg) * H % 2 == 1 for i in range(1, segments))
    d = make_inputs_device(B, T, H, dd, dd, seed=107 + dd, device=cuda, h0_std=0.02)
    if prec == "fp16":
        d.update({n: d[n].to(torch.float16) for n in ("q", "k", "v", "g", "beta")})
    elif prec == "bf16_f32gates":
        d.update({n: d[n].float() for n in ("g", "beta")})
    print(f"[full] overlapped segments d={dd} {prec}", flush=True)
    o, ht = _fwd(d, h0=d["h0"])
    x = _host(d)
    o_ref, ht_ref = K.chunk_fwd(x["q"], x["k"], x["v"], x["g"], x["beta"], h0=d["h0"].cpu().numpy(), chunk=64)
    tol = TOL["fp16" if prec == "fp16" else "bf16"]
    assert_chains_close("o", o, o_ref, tol, chain_axes=(0, 2))
    assert_chains_close("ht", ht, ht_ref, tol, chain_axes=(0, 1))
    half = 64 * 781
    o1, h1 = _fwd(_slice(d, 0, half), h0=d["h0"])
    o2, h2 = _fwd(_slice(d, half, T), h0=h1)
    assert torch.equal(torch.cat([o1, o2], dim=1), o) and torch.equal(h2, ht)
    ob, _ = axiom_amd.kda_chunk_fwd(d["q"], d["k"], d["v"], d["g"], d["beta"], initial_state=d["h0"],
                                    out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.equal(ob, o.to(torch.bfloat16))
