"""GPU parity under strong decay: g scaled so that a 16-row tile's total decay
reaches 2^-130 in some channels (the forward's intra kernel then takes its
mid-tile-anchored path; the backward's anchored factors and per-element
diagonal exponentials see products near the fp32 range's ends).

Same bars as the ordinary cases: forward o and final state rel-L2 <= 1e-3 and
max-abs <= 2e-2 (bf16 inputs), <= 1e-5 (fp32, exact mode); backward every
gradient rel-L2 <= 1e-4 and max-abs <= 1e-4 x max|reference| (fp32 inputs),
<= 1e-3 and <= 2e-3 x max|reference| (bf16 inputs: the 16-bit workspace of
tests/test_gpu_bwd.py) against the float64 oracle on the same inputs.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import inputs, kda_oracle as K
from tests.kda_testutil import TDT, TOL, assert_close, to_dev

pytestmark = pytest.mark.gpu

G_SCALE = 8.0   # |g| up to ~30 per step; a 16-row tile up to ~2^-130 per channel


def _strong(B, T, H, d, seed, dtype):
    x = inputs.make_inputs(B, T, H, d, d, seed=seed, dtype="fp32", h0_std=0.05)
    x["g"] = (x["g"] * np.float32(G_SCALE)).astype(np.float32)
    if dtype == "bf16":
        for n in ("q", "k", "v", "g", "beta"):
            x[n] = inputs.bf16_round(x[n])
    return x


def test_strong_decay_reaches_the_extreme_tiles():
    """The inputs do what the tests below rely on: some tile's total decay passes 2^-100."""
    x = _strong(2, 256, 4, 128, seed=21, dtype="bf16")
    g = x["g"].reshape(2, 16, 16, 4, 128)                 # [B, tiles, 16 rows, H, d]
    tile_log2 = g.sum(axis=2) / np.log(2.0)
    assert tile_log2.min() < -100.0
    assert np.isfinite(K.chunk_fwd(x["q"][:, :64], x["k"][:, :64], x["v"][:, :64], x["g"][:, :64],
                                   x["beta"][:, :64], chunk=64)[0].numpy()).all()


@pytest.mark.parametrize("prec,d", [("bf16", 128), ("bf16", 64), ("fp32", 64)])
def test_forward_strong_decay(cuda, prec, d):
    import axiom_amd
    x = _strong(2, 256, 4, d, seed=21 + d, dtype=prec)
    dt = TDT[prec]
    ts = [to_dev(x[n], dt, cuda) for n in ("q", "k", "v", "g", "beta")]
    h0 = to_dev(x["h0"], torch.float32, cuda)
    print(f"[strong decay fwd] {prec} d={d}", flush=True)
    o, ht = axiom_amd.kda_chunk_fwd(*ts, initial_state=h0)
    torch.cuda.synchronize()
    o_ref, ht_ref = K.chunk_fwd(x["q"], x["k"], x["v"], x["g"], x["beta"], h0=x["h0"], chunk=64)
    assert_close("o", o, o_ref, TOL[prec])
    assert_close("ht", ht, ht_ref, TOL[prec])


@pytest.mark.parametrize("prec,d", [("bf16", 128), ("bf16", 64), ("fp32", 64)])
def test_forward_decay_spikes(cuda, prec, d):
    """Single steps that decay by e^-150 (2^-216, past fp32's range in one
    factor) in 3 % of the gate entries: the extreme tiles' pairs go through
    anchors between their rows, so o and the final state stay finite and on
    the oracle."""
    import axiom_amd
    x = inputs.make_inputs(2, 192, 2, d, d, seed=41 + d, dtype="fp32", h0_std=0.05)
    rng = np.random.default_rng(41 + d)
    x["g"] = np.where(rng.random(x["g"].shape) < 0.03, np.float32(-150.0), x["g"]).astype(np.float32)
    if prec == "bf16":
        for n in ("q", "k", "v", "g", "beta"):
            x[n] = inputs.bf16_round(x[n])
    dt = TDT[prec]
    ts = [to_dev(x[n], dt, cuda) for n in ("q", "k", "v", "g", "beta")]
    h0 = to_dev(x["h0"], torch.float32, cuda)
    print(f"[decay spikes fwd] {prec} d={d}", flush=True)
    o, ht = axiom_amd.kda_chunk_fwd(*ts, initial_state=h0)
    torch.cuda.synchronize()
    assert torch.isfinite(o).all() and torch.isfinite(ht).all()
    # the token-by-token oracle: the chunked one forms e^(G_c - G_i) from
    # e^G and e^-G, which leave float64's range once a channel's decay within
    # a chunk passes e^-709 (a few spikes in one channel)
    o_ref, ht_ref = K.recurrent_fwd(x["q"], x["k"], x["v"], x["g"], x["beta"], h0=x["h0"])
    assert_close("o", o, o_ref, TOL[prec])
    assert_close("ht", ht, ht_ref, TOL[prec])


@pytest.mark.parametrize("prec,d,T", [("bf16", 128, 192), ("fp32", 64, 192), ("bf16", 64, 150)])
def test_backward_strong_decay(cuda, prec, d, T):
    # (T = 150: a ragged last chunk, whose pad rows the chunk kernel's
    # in-kernel cumsum of g must treat as zero decay)
    import axiom_amd
    x = _strong(1, T, 2, d, seed=31 + d, dtype=prec)
    rng = np.random.default_rng(5)
    do = rng.standard_normal((1, T, 2, d)).astype(np.float32)
    dS = (rng.standard_normal((1, 2, d, d)) * 0.1).astype(np.float32)
    dt = TDT[prec]
    ts = [to_dev(x[n], dt, cuda) for n in ("q", "k", "v", "g", "beta")]
    print(f"[strong decay bwd] {prec} d={d} T={T}", flush=True)
    got = axiom_amd.kda_chunk_bwd(*ts, to_dev(do, torch.float32, cuda), dht=to_dev(dS, torch.float32, cuda),
                                  initial_state=to_dev(x["h0"], torch.float32, cuda))
    torch.cuda.synchronize()
    ref = K.chunk_bwd(*(x[n].astype(np.float64) for n in ("q", "k", "v", "g", "beta")), do.astype(np.float64),
                      dht=dS.astype(np.float64), h0=x["h0"], chunk=64)
    for name, a, b in zip(("dq", "dk", "dv", "dg", "dbeta", "dh0"), got, ref):
        a = a.double().cpu().numpy()
        assert np.all(np.isfinite(a)), name
        rel, mx = K.rel_l2(a, b), K.max_abs(a, b)
        print(f"  {name}: rel_l2={rel:.2e} max_abs={mx:.2e}", flush=True)
        rt, at = (1e-4, 1e-4) if prec == "fp32" else (1e-3, 2e-3)
        assert rel <= rt and mx <= at * max(1.0, float(np.abs(b).max())), (name, rel, mx)
