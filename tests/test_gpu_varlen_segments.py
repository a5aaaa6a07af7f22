"""GPU parity of segmented varlen calls.

A varlen call given less workspace than its fastest schedule needs (at least
kda_chunk_fwd_workspace_min) runs in segments of a position-major unit
numbering (every sequence's chunk p before any sequence's chunk p + 1,
sequences longest-first), the largest that fit; each chain's state crosses
the segment boundaries in the final-state buffer (or, when no final state is
asked for, in a workspace copy).  Many heads make small calls segmented here
(the budget is per call, over all heads), so the cases below run in 2-3
segments with the column state kernel (d = 64), the whole-chain state kernel
(d = 128, at least 256 chains) and exact mode (fp32).

Checked: the segmented call equals the unsegmented one (full workspace) bit
for bit, and so does a call with a workspace between the two sizes; every
(sequence, head) chain against the fp64 oracle, each on its own (the bf16
bar, or fp32's); the packed call equals each sequence's own dense call bit
for bit (the state crosses segments in fp32, as it crosses chunks); the call
without a final state gives the same o bit for bit; empty and one-token
sequences keep h0 and get their one row.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import inputs, kda_oracle as K
from tests.kda_testutil import TDT, TOL, assert_chain_errors, assert_chains_close, chain_errors, to_dev
from tests.test_capi import varlen_segments

pytestmark = pytest.mark.gpu

_CODES = {"bf16": 1, "fp32": 0}


def _min_ws(cuda, T, N, H, d, prec, extra=0):
    from axiom_amd import kda as kmod
    n = kmod.chunk_fwd_workspace_min_bytes(1, T, H, d, d, n_seqs=N, in_code=_CODES[prec])
    return torch.empty(n + extra, dtype=torch.uint8, device=cuda)

CASES = [
    # lengths, H, d, precision
    ([900, 0, 1, 640, 130, 2000, 64, 65], 128, 64, "bf16"),
    ([1200, 700, 5, 0, 333, 800, 64], 64, 128, "bf16"),
    ([500, 1, 0, 300, 640], 128, 64, "fp32"),
]


@pytest.mark.parametrize("lengths,H,d,prec", CASES)
def test_segmented_varlen_matches_oracle_and_per_sequence(cuda, lengths, H, d, prec):
    import axiom_amd
    N = len(lengths)
    cu = inputs.cu_seqlens_from_lengths(lengths)
    T = int(cu[-1])
    es = 4 if prec == "fp32" else 2
    segs, ku = varlen_segments(T, N, H, d, d, es)
    assert segs > 1, "the case must run segmented"
    x = inputs.make_inputs(1, T, H, d, d, seed=T + H + d, dtype="fp32" if prec == "fp32" else "bf16",
                           h0_std=0.05, n_states=N)
    dt = TDT[prec]
    ts = [to_dev(x[n], dt, cuda) for n in ("q", "k", "v", "g", "beta")]
    h0 = to_dev(x["h0"], torch.float32, cuda)
    cu_t = torch.from_numpy(cu).to(cuda)
    print(f"[varlen segments] lengths={lengths} H={H} d={d} {prec}: {segs} segments of {ku} units", flush=True)
    ws = _min_ws(cuda, T, N, H, d, prec)
    o, ht = axiom_amd.kda_chunk_fwd(*ts, initial_state=h0, cu_seqlens=cu_t, workspace=ws)
    o_nf, ht_nf = axiom_amd.kda_chunk_fwd(*ts, initial_state=h0, cu_seqlens=cu_t, output_final_state=False,
                                          workspace=ws)
    o_full, ht_full = axiom_amd.kda_chunk_fwd(*ts, initial_state=h0, cu_seqlens=cu_t)
    o_mid, ht_mid = axiom_amd.kda_chunk_fwd(*ts, initial_state=h0, cu_seqlens=cu_t,
                                            workspace=_min_ws(cuda, T, N, H, d, prec, extra=40 << 20))
    torch.cuda.synchronize()
    assert ht_nf is None and torch.equal(o_nf, o)
    assert torch.equal(o, o_full) and torch.equal(ht, ht_full), "segmented != unsegmented"
    assert torch.equal(o, o_mid) and torch.equal(ht, ht_mid), "larger segments differ"
    # every chain against the oracle
    o_ref, ht_ref = K.chunk_fwd(x["q"], x["k"], x["v"], x["g"], x["beta"], h0=x["h0"], cu_seqlens=cu, chunk=64)
    o_np, o_ref = o.double().cpu().numpy(), o_ref.numpy()
    rel, mx = [], []
    for i in range(N):
        a, b = int(cu[i]), int(cu[i + 1])
        if b > a:
            r_, m_ = chain_errors(o_np[:, a:b], o_ref[:, a:b], chain_axes=(2,))
            rel.append(r_)
            mx.append(m_)
    assert_chain_errors("o", np.stack(rel), np.stack(mx), TOL[prec])
    assert_chains_close("ht", ht, ht_ref, TOL[prec], chain_axes=(0, 1))
    # each sequence's own dense call, bit for bit; an empty one keeps h0
    for i in range(N):
        a, b = int(cu[i]), int(cu[i + 1])
        if b == a:
            assert torch.equal(ht[i], h0[i]), f"sequence {i} (empty): final state is not h0"
            continue
        oi, hi = axiom_amd.kda_chunk_fwd(*(t[:, a:b].contiguous() for t in ts), initial_state=h0[i:i + 1].contiguous())
        torch.cuda.synchronize()
        assert torch.equal(oi, o[:, a:b]), f"sequence {i}: packed o differs from its own run"
        assert torch.equal(hi[0], ht[i]), f"sequence {i}: packed state differs from its own run"


def test_segmented_varlen_without_h0(cuda):
    """No initial state (zeros) and a final state: equal to the call with an
    all-zero h0, bit for bit."""
    import axiom_amd
    lengths, H, d = [700, 64, 1, 1500, 0, 260], 128, 64
    N = len(lengths)
    cu = inputs.cu_seqlens_from_lengths(lengths)
    T = int(cu[-1])
    assert varlen_segments(T, N, H, d, d, 2)[0] > 1
    x = inputs.make_inputs(1, T, H, d, d, seed=77, dtype="bf16")
    ts = [to_dev(x[n], torch.bfloat16, cuda) for n in ("q", "k", "v", "g", "beta")]
    cu_t = torch.from_numpy(cu).to(cuda)
    print("[varlen segments] no h0", flush=True)
    ws = _min_ws(cuda, T, N, H, d, "bf16")
    o, ht = axiom_amd.kda_chunk_fwd(*ts, cu_seqlens=cu_t, workspace=ws)
    o0, ht0 = axiom_amd.kda_chunk_fwd(*ts, cu_seqlens=cu_t, workspace=ws,
                                      initial_state=torch.zeros(N, H, d, d, device=cuda))
    torch.cuda.synchronize()
    assert torch.equal(o, o0) and torch.equal(ht, ht0)
    assert torch.count_nonzero(ht[4]) == 0
