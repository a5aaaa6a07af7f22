"""GPU parity of the HIP KDA path against the CPU oracle (small, seeded cases).

Every case calls the C ABI through ``axiom_amd`` on ``cuda:0`` and compares o
and the final state with the fp64 oracle on the same (bf16-rounded) inputs:
rel-L2 <= 1e-3 and max-abs <= 2e-2 for bf16/fp16 inputs, both <= 1e-5 for
fp32 inputs (exact mode).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import inputs, kda_oracle as K
from tests.kda_testutil import TDT, TOL, assert_close, to_dev

pytestmark = pytest.mark.gpu


def _run_chunk(cuda, d, prec, h0=None, cu=None, scale=1.0, gates_fp32=False, out_dtype=torch.float32):
    import axiom_amd
    dt = TDT[prec]
    gdt = torch.float32 if gates_fp32 else dt
    q, k, v = (to_dev(d[n], dt, cuda) for n in ("q", "k", "v"))
    g = to_dev(d["g"], gdt, cuda)
    beta = to_dev(d["beta"], gdt, cuda)
    h0_t = None if h0 is None else to_dev(h0, torch.float32, cuda)
    cu_t = None if cu is None else torch.from_numpy(np.asarray(cu, np.int32)).to(cuda)
    o, ht = axiom_amd.kda_chunk_fwd(q, k, v, g, beta, initial_state=h0_t, cu_seqlens=cu_t,
                                    scale=scale, out_dtype=out_dtype)
    torch.cuda.synchronize()
    return o, ht


def _oracle(d, h0=None, cu=None, scale=1.0):
    return K.chunk_fwd(d["q"], d["k"], d["v"], d["g"], d["beta"], h0=h0, cu_seqlens=cu,
                       chunk=64, scale=scale)


def test_config0_fp32_exact(cuda):
    """Config 0 shape (B1 T512 H4 d64, fp32): exact mode, 1e-5 bar."""
    d = inputs.make_inputs(1, 512, 4, 64, 64, seed=0, dtype="fp32")
    o, ht = _run_chunk(cuda, d, "fp32")
    o_ref, ht_ref = _oracle(d)
    assert_close("o", o, o_ref, TOL["fp32"])
    assert_close("ht", ht, ht_ref, TOL["fp32"])


@pytest.mark.parametrize("dk", [64, 128])
def test_bf16_dense(cuda, dk):
    d = inputs.make_inputs(2, 256, 4, dk, dk, seed=1, dtype="bf16")
    o, ht = _run_chunk(cuda, d, "bf16")
    o_ref, ht_ref = _oracle(d)
    assert_close("o", o, o_ref, TOL["bf16"])
    assert_close("ht", ht, ht_ref, TOL["bf16"])


@pytest.mark.parametrize("T", [1, 17, 63, 64, 65, 130, 191])
def test_ragged_T(cuda, T):
    d = inputs.make_inputs(2, T, 3, 128, 128, seed=T, dtype="bf16", h0_std=0.02)
    o, ht = _run_chunk(cuda, d, "bf16", h0=d["h0"])
    o_ref, ht_ref = _oracle(d, h0=d["h0"])
    assert_close("o", o, o_ref, TOL["bf16"])
    assert_close("ht", ht, ht_ref, TOL["bf16"])


@pytest.mark.parametrize("T", [1, 40, 64, 100])
def test_ragged_T_fp32(cuda, T):
    d = inputs.make_inputs(1, T, 2, 64, 64, seed=T, dtype="fp32", h0_std=0.1)
    o, ht = _run_chunk(cuda, d, "fp32", h0=d["h0"])
    o_ref, ht_ref = _oracle(d, h0=d["h0"])
    assert_close("o", o, o_ref, TOL["fp32"])
    assert_close("ht", ht, ht_ref, TOL["fp32"])


def test_fp16_inputs(cuda):
    d = inputs.make_inputs(1, 320, 4, 128, 128, seed=5, dtype="fp32")
    for n in ("q", "k", "v", "g", "beta"):
        d[n] = d[n].astype(np.float16).astype(np.float32)
    o, ht = _run_chunk(cuda, d, "fp16")
    o_ref, ht_ref = _oracle(d)
    assert_close("o", o, o_ref, TOL["fp16"])
    assert_close("ht", ht, ht_ref, TOL["fp16"])


@pytest.mark.parametrize("T,dk", [(256, 128), (200, 128), (200, 64)])
def test_bf16_with_fp32_gates(cuda, T, dk):
    # fp32 gate rows are staged through LDS like the 16-bit rows (a ragged T
    # re-reads the last row for the rows past the end)
    d = inputs.make_inputs(1, T, 4, dk, dk, seed=6, dtype="bf16")
    d["g"] = (d["g"] * np.float32(0.9731)).astype(np.float32)   # not bf16-representable
    o, ht = _run_chunk(cuda, d, "bf16", gates_fp32=True)
    o_ref, ht_ref = _oracle(d)
    assert_close("o", o, o_ref, TOL["bf16"])
    assert_close("ht", ht, ht_ref, TOL["bf16"])


def test_scale_and_bf16_output(cuda):
    d = inputs.make_inputs(1, 200, 2, 128, 128, seed=7, dtype="bf16")
    o, ht = _run_chunk(cuda, d, "bf16", scale=0.5, out_dtype=torch.bfloat16)
    o_ref, ht_ref = _oracle(d, scale=0.5)
    assert o.dtype == torch.bfloat16
    assert_close("o", o, o_ref, (4e-3, 2e-2))   # includes the bf16 rounding of o itself
    assert_close("ht", ht, ht_ref, TOL["bf16"])


@pytest.mark.parametrize("prec", ["bf16", "fp32"])
def test_varlen(cuda, prec):
    lengths = [1, 64, 100, 0, 200, 63, 65, 130]
    cu = inputs.cu_seqlens_from_lengths(lengths)
    T = int(cu[-1])
    dk = 128 if prec == "bf16" else 64
    d = inputs.make_inputs(1, T, 4, dk, dk, seed=11, dtype=prec, h0_std=0.02,
                           n_states=len(lengths))
    o, ht = _run_chunk(cuda, d, prec, h0=d["h0"], cu=cu)
    o_ref, ht_ref = _oracle(d, h0=d["h0"], cu=cu)
    assert_close("o", o, o_ref, TOL[prec])
    assert_close("ht", ht, ht_ref, TOL[prec])


def test_varlen_equals_per_sequence_runs(cuda):
    """Packed run == independent runs of each sequence (GPU against GPU)."""
    lengths = [70, 5, 128, 33]
    cu = inputs.cu_seqlens_from_lengths(lengths)
    d = inputs.make_inputs(1, int(cu[-1]), 2, 128, 128, seed=12, dtype="bf16", h0_std=0.02,
                           n_states=len(lengths))
    o, ht = _run_chunk(cuda, d, "bf16", h0=d["h0"], cu=cu)
    for i in range(len(lengths)):
        a, b = int(cu[i]), int(cu[i + 1])
        di = {n: d[n][:, a:b] for n in ("q", "k", "v", "g", "beta")}
        oi, hi = _run_chunk(cuda, di, "bf16", h0=d["h0"][i:i + 1])
        np.testing.assert_array_equal(o[:, a:b].cpu().numpy(), oi.cpu().numpy())
        np.testing.assert_array_equal(ht[i].cpu().numpy(), hi[0].cpu().numpy())


def test_cc_scan_seam(cuda):
    """The reference seam: alpha/beta32 operands, (T, H*d) layouts, functional S."""
    import axiom_amd
    T, H, d = 192, 4, 128
    dd = inputs.make_inputs(1, T, H, d, d, seed=13, dtype="bf16", h0_std=0.05)
    alpha = np.exp(dd["g"].astype(np.float64)).astype(np.float32)
    g_eff = np.log(alpha.astype(np.float64)).astype(np.float32)
    beta32 = np.repeat(dd["beta"][..., None], 32, axis=-1).reshape(T, H * 32)
    q = to_dev(dd["q"].reshape(T, H * d), torch.bfloat16, cuda)
    k = to_dev(dd["k"].reshape(T, H * d), torch.bfloat16, cuda)
    v = to_dev(dd["v"].reshape(T, H * d), torch.bfloat16, cuda)
    S = to_dev(dd["h0"][0], torch.float32, cuda)
    S_before = S.clone()
    o, S_new = axiom_amd.cc_scan(q, k, v, to_dev(alpha.reshape(T, H * d), torch.float32, cuda),
                                 to_dev(beta32, torch.float32, cuda), S, tile=16, chunk=32)
    torch.cuda.synchronize()
    assert torch.equal(S, S_before)
    o_ref, s_ref = K.chunk_fwd(dd["q"], dd["k"], dd["v"], g_eff, dd["beta"], h0=dd["h0"], chunk=64)
    assert_close("o", o.reshape(1, T, H, d), o_ref, TOL["bf16"])
    assert_close("S_new", S_new, s_ref[0], TOL["bf16"])


def test_cc_scan_seam_denormal_alpha(cuda):
    """Denormal alpha values (a gate that has decayed past fp32's normal
    range) are finite log-decays of -87 to -103, as in the oracle: the
    forward must not turn them into -inf (and NaN factors)."""
    import axiom_amd
    T, H, d = 128, 2, 128
    dd = inputs.make_inputs(1, T, H, d, d, seed=14, dtype="bf16", h0_std=0.05)
    alpha = np.exp(dd["g"].astype(np.float64)).astype(np.float32)
    rng = np.random.default_rng(14)
    pick = rng.random(alpha.shape) < 0.02
    alpha[pick] = rng.uniform(1e-44, 1e-38, size=int(pick.sum())).astype(np.float32)
    assert (alpha[pick] < np.finfo(np.float32).tiny).all() and (alpha > 0).all()
    g_eff = np.log(alpha.astype(np.float64)).astype(np.float32)
    beta32 = np.repeat(dd["beta"][..., None], 32, axis=-1).reshape(T, H * 32)
    q, k, v = (to_dev(dd[n].reshape(T, H * d), torch.bfloat16, cuda) for n in ("q", "k", "v"))
    S = to_dev(dd["h0"][0], torch.float32, cuda)
    o, S_new = axiom_amd.cc_scan(q, k, v, to_dev(alpha.reshape(T, H * d), torch.float32, cuda),
                                 to_dev(beta32, torch.float32, cuda), S, tile=16, chunk=32)
    torch.cuda.synchronize()
    assert torch.isfinite(o).all() and torch.isfinite(S_new).all()
    o_ref, s_ref = K.chunk_fwd(dd["q"], dd["k"], dd["v"], g_eff, dd["beta"], h0=dd["h0"], chunk=64)
    assert_close("o", o.reshape(1, T, H, d), o_ref, TOL["bf16"])
    assert_close("S_new", S_new, s_ref[0], TOL["bf16"])


def test_cc_scan_errors(cuda):
    import axiom_amd
    T, H, d = 96, 2, 128
    z = torch.zeros((T, H * d), device=cuda)
    with pytest.raises(ValueError, match="multiple of the chunk width"):
        axiom_amd.cc_scan(z.bfloat16(), z.bfloat16(), z.bfloat16(), z, torch.zeros((T, H * 32), device=cuda),
                          torch.zeros((H, d, d), device=cuda), chunk=64)
    with pytest.raises(ValueError, match="bf16"):
        axiom_amd.cc_scan(z, z, z, z, torch.zeros((T, H * 32), device=cuda),
                          torch.zeros((H, d, d), device=cuda), chunk=32)


@pytest.mark.parametrize("prec,dk", [("bf16", 128), ("fp32", 64), ("fp16", 128)])
def test_decode_step(cuda, prec, dk):
    import axiom_amd
    B, H, steps = 8, 4, 3
    d = inputs.make_decode_inputs(B, H, dk, dk, steps, seed=21, dtype="bf16" if prec == "bf16" else "fp32")
    if prec == "fp16":
        for n in ("q", "k", "v", "g", "beta"):
            d[n] = d[n].astype(np.float16).astype(np.float32)
    dt = TDT[prec]
    S = to_dev(d["S"], torch.float32, cuda)
    S_ref = d["S"].astype(np.float64)
    for t in range(steps):
        o = axiom_amd.kda_recurrent_step(*(to_dev(d[n][t], dt, cuda) for n in ("q", "k", "v", "g", "beta")), S)
        o_ref, S_ref = K.decode_step(d["q"][t], d["k"][t], d["v"][t], d["g"][t], d["beta"][t], S_ref)
        torch.cuda.synchronize()
        assert_close(f"o[{t}]", o, o_ref, (1e-5, 1e-5))
    assert_close("S", S, S_ref, (1e-5, 1e-5))


def test_decode_matches_chunked(cuda):
    """T decode steps == chunked forward over the same T tokens (GPU vs GPU)."""
    import axiom_amd
    B, T, H, dk = 2, 70, 2, 128
    d = inputs.make_inputs(B, T, H, dk, dk, seed=22, dtype="bf16", h0_std=0.02)
    o_c, ht_c = _run_chunk(cuda, d, "bf16", h0=d["h0"])
    S = to_dev(d["h0"], torch.float32, cuda)
    outs = []
    for t in range(T):
        outs.append(axiom_amd.kda_recurrent_step(
            *(to_dev(d[n][:, t], torch.bfloat16, cuda) for n in ("q", "k", "v", "g", "beta")), S))
    o_d = torch.stack(outs, 1)
    torch.cuda.synchronize()
    assert_close("o", o_c, o_d.cpu().double(), TOL["bf16"])
    assert_close("ht", ht_c, S.cpu().double(), TOL["bf16"])
