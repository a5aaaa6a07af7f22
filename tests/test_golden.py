"""Golden fixtures (``tests/golden/*.npz``): the CPU side and the GPU side.

CPU (unmarked): the input generator still draws the frozen inputs bit for
bit, the float64 recurrence still produces the frozen outputs, and the chunked
oracle agrees with them, so a change to either oracle form is caught against
data that does not move.

GPU (``gpu``): the HIP path on the frozen inputs against the frozen outputs,
at the north-star bar for the input precision.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import inputs, kda_oracle as K
from tests.golden.make_golden import CASES, load
from tests.kda_testutil import TDT, TOL, assert_close, to_dev

DENSE = ["dense_fp32_d64", "dense_bf16_d128_h0"]


def test_every_fixture_present():
    for name in CASES:
        load(name)


@pytest.mark.parametrize("name", DENSE + ["varlen_bf16_d64"])
def test_generator_reproduces_inputs(name):
    f = load(name)
    B, T, H, dk, seed = (int(x) for x in f["meta"])
    kw = {}
    if "h0" in f:
        kw = dict(h0_std=0.02, n_states=f["h0"].shape[0])
    d = inputs.make_inputs(B, T, H, dk, dk, seed=seed, dtype=f["prec"], **kw)
    for key in ("q", "k", "v", "g", "beta") + (("h0",) if "h0" in f else ()):
        assert np.array_equal(d[key], f[key]), key


@pytest.mark.parametrize("name", DENSE + ["varlen_bf16_d64"])
def test_recurrence_reproduces_fixture(name):
    f = load(name)
    o, ht = K.recurrent_fwd(f["q"], f["k"], f["v"], f["g"], f["beta"], h0=f.get("h0"),
                            cu_seqlens=f.get("cu_seqlens"))
    # stored as float32: agreement to float32 rounding
    assert K.rel_l2(o, f["o"]) < 1e-7 and K.rel_l2(ht, f["ht"]) < 1e-7


@pytest.mark.parametrize("name", DENSE + ["varlen_bf16_d64"])
def test_chunked_oracle_matches_fixture(name):
    f = load(name)
    o, ht = K.chunk_fwd(f["q"], f["k"], f["v"], f["g"], f["beta"], h0=f.get("h0"),
                        cu_seqlens=f.get("cu_seqlens"), chunk=64)
    assert K.rel_l2(o.numpy(), f["o"]) < 1e-7
    assert K.rel_l2(ht.numpy(), f["ht"]) < 1e-7


def test_decode_fixture():
    f = load("decode_bf16_d64")
    B, H, dk, steps, seed = (int(x) for x in f["meta"])
    d = inputs.make_decode_inputs(B, H, dk, dk, steps, seed=seed, dtype="bf16")
    assert np.array_equal(d["S"], f["S0"])
    o, S = K.decode_steps(f["q"], f["k"], f["v"], f["g"], f["beta"], f["S0"])
    assert K.rel_l2(o, f["o"]) < 1e-7 and K.rel_l2(S, f["S"]) < 1e-7


# ---------------------------------------------------------------------------
# GPU: HIP path against the frozen outputs
# ---------------------------------------------------------------------------


@pytest.mark.gpu
@pytest.mark.parametrize("name", DENSE + ["varlen_bf16_d64"])
def test_gpu_chunk_fwd_matches_fixture(cuda, name):
    import axiom_amd
    f = load(name)
    dt = TDT[f["prec"]]
    q, k, v, g, beta = (to_dev(f[n], dt, cuda) for n in ("q", "k", "v", "g", "beta"))
    h0 = to_dev(f["h0"], torch.float32, cuda) if "h0" in f else None
    cu = torch.from_numpy(f["cu_seqlens"]).to(cuda) if "cu_seqlens" in f else None
    print(f"[golden] {name}", flush=True)
    o, ht = axiom_amd.kda_chunk_fwd(q, k, v, g, beta, initial_state=h0, cu_seqlens=cu)
    torch.cuda.synchronize()
    assert_close("o", o, f["o"], TOL[f["prec"]])
    assert_close("ht", ht, f["ht"], TOL[f["prec"]])


@pytest.mark.gpu
def test_gpu_decode_matches_fixture(cuda):
    import axiom_amd
    f = load("decode_bf16_d64")
    S = to_dev(f["S0"], torch.float32, cuda)
    outs = []
    for t in range(f["q"].shape[0]):
        step = [to_dev(f[n][t], torch.bfloat16, cuda) for n in ("q", "k", "v", "g", "beta")]
        outs.append(axiom_amd.kda_recurrent_step(*step, S))
    torch.cuda.synchronize()
    assert_close("o", torch.stack(outs), f["o"], (1e-5, 1e-5))
    assert_close("S", S, f["S"], (1e-5, 1e-5))
