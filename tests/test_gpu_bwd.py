"""GPU parity of the chunked backward (kda_chunk_bwd) against the fp64 oracle.

The oracle's adjoint is pinned on the CPU (tests/test_oracle_bwd.py: finite
differences, autograd of an independent recurrence).  Here the HIP backward
runs on the same (dtype-rounded) inputs and cotangents and every gradient --
dq, dk, dv, dg, dbeta, dh0 -- is compared with it.

fp32 inputs: the backward computes in fp32 throughout; relative L2 error
<= 1e-4 and max-abs error <= 1e-4 x max|reference| per gradient (measured
~5e-6).  16-bit inputs store six forward-side workspace arrays in fp16 (the
forward kernels' operand width; oracle/emulate_bwd.py lists them): against the
float64 oracle the bf16 bar of the forward, relative L2 <= 1e-3, with max-abs
<= 2e-3 x max|reference| (measured <= 2.3e-4 and 3.1e-4), and against the
rounding-point emulation of those arrays relative L2 <= 1e-4, max-abs <=
5e-4 x max|reference| (measured <= 2.6e-5 and 1.1e-4): the kernels land on
the emulated roundings, not merely inside the bar.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import emulate_bwd as EB
from oracle import inputs, kda_oracle as K
from tests.kda_testutil import TDT, to_dev

pytestmark = pytest.mark.gpu

NAMES = ("dq", "dk", "dv", "dg", "dbeta", "dh0")
REL = 1e-4                      # fp32 inputs (relative L2 and max-abs / max|ref|)
REL16, ABS16 = 1e-3, 2e-3       # 16-bit inputs against the float64 oracle
EREL16, EABS16 = 1e-4, 5e-4     # 16-bit inputs against the rounding emulation


def _case(B, T, H, d, seed, prec, h0=True, dht=True):
    x = inputs.make_inputs(B, T, H, d, d, seed=seed, dtype="bf16" if prec != "fp32" else "fp32",
                           h0_std=0.05 if h0 else 0.0)
    rng = np.random.default_rng(seed + 1)
    do = rng.standard_normal((B, T, H, d)).astype(np.float32)
    dS = rng.standard_normal((B, H, d, d)).astype(np.float32) * 0.1 if dht else None
    return x, do, dS


def _hip(cuda, x, do, dS, prec, scale=1.0, do_bf16=False):
    import axiom_amd
    dt = TDT[prec]
    q, k, v, g, beta = (to_dev(x[n], dt, cuda) for n in ("q", "k", "v", "g", "beta"))
    h0 = to_dev(x["h0"], torch.float32, cuda) if "h0" in x else None
    do_t = to_dev(do, torch.bfloat16 if do_bf16 else torch.float32, cuda)
    dht = None if dS is None else to_dev(dS, torch.float32, cuda)
    out = axiom_amd.kda_chunk_bwd(q, k, v, g, beta, do_t, dht=dht, initial_state=h0, scale=scale)
    torch.cuda.synchronize()
    return dict(zip(NAMES, out))


def _as(a, dt):
    """The values a tensor of dtype dt holds for the float32 array a (what the GPU sees)."""
    return torch.from_numpy(np.ascontiguousarray(a)).to(dt).double().numpy()


def _ref(x, do, dS, scale=1.0, prec="fp32", do_bf16=False, emulate=False):
    xs = {n: _as(x[n], TDT[prec]) for n in ("q", "k", "v", "g", "beta")}
    do_r = _as(do, torch.bfloat16 if do_bf16 else torch.float32)
    fn = EB.emulate_bwd if emulate else K.chunk_bwd
    kw = {} if emulate else {"chunk": 64}
    out = fn(xs["q"], xs["k"], xs["v"], xs["g"], xs["beta"], do_r.astype(np.float64),
             dht=None if dS is None else dS.astype(np.float64), h0=x.get("h0"), scale=scale, **kw)
    return dict(zip(NAMES, out))


def _check(got, ref, rel_tol=REL, abs_tol=REL, tag=""):
    msgs = []
    for n in NAMES:
        if ref[n] is None or got[n] is None:
            continue
        a = got[n].float().cpu().numpy().astype(np.float64)
        b = ref[n]
        assert a.shape == b.shape, (n, a.shape, b.shape)
        assert np.all(np.isfinite(a)), f"{n}: non-finite"
        rel = K.rel_l2(a, b)
        mx = K.max_abs(a, b)
        scale = max(1.0, float(np.abs(b).max()))
        msgs.append(f"{n}: rel_l2={rel:.2e} max_abs={mx:.2e}")
        assert rel <= rel_tol and mx <= abs_tol * scale, tag + "; ".join(msgs)
    print(tag + " | ".join(msgs), flush=True)


def _check_all(got, x, do, dS, scale=1.0, prec="fp32", do_bf16=False):
    """fp32: the 1e-4 bar against the oracle; 16-bit: the bf16 bar against the
    oracle and the tight bar against the rounding emulation."""
    if prec == "fp32":
        _check(got, _ref(x, do, dS, scale, prec, do_bf16))
        return
    _check(got, _ref(x, do, dS, scale, prec, do_bf16), REL16, ABS16, "oracle: ")
    _check(got, _ref(x, do, dS, scale, prec, do_bf16, emulate=True), EREL16, EABS16, "emulation: ")


@pytest.mark.parametrize("B,T,H,d,prec,scale", [
    (1, 128, 2, 64, "fp32", 1.0),
    (1, 64, 1, 128, "bf16", 1.0),
    (2, 200, 2, 128, "bf16", 0.8),
    (1, 100, 3, 64, "fp16", 1.0),
    (1, 1, 2, 128, "bf16", 1.0),
])
def test_bwd_matches_oracle(cuda, B, T, H, d, prec, scale):
    x, do, dS = _case(B, T, H, d, seed=T + d, prec=prec)
    print(f"[bwd] B={B} T={T} H={H} d={d} {prec} scale={scale}", flush=True)
    got = _hip(cuda, x, do, dS, prec, scale)
    _check_all(got, x, do, dS, scale, prec)


def test_bwd_without_initial_state_or_state_cotangent(cuda):
    x, do, dS = _case(1, 130, 2, 128, seed=4, prec="bf16", h0=False, dht=False)
    got = _hip(cuda, x, do, None, "bf16")
    _check_all(got, x, do, None, 1.0, "bf16")


def test_bwd_bf16_output_cotangent(cuda):
    x, do, dS = _case(1, 96, 2, 64, seed=6, prec="bf16")
    got = _hip(cuda, x, do, dS, "bf16", do_bf16=True)
    _check_all(got, x, do, dS, 1.0, "bf16", do_bf16=True)


def test_bwd_empty_sequence_passes_the_state_cotangent(cuda):
    import axiom_amd
    dev = cuda
    q = torch.zeros((1, 0, 2, 64), dtype=torch.bfloat16, device=dev)
    v = torch.zeros((1, 0, 2, 64), dtype=torch.bfloat16, device=dev)
    beta = torch.zeros((1, 0, 2), dtype=torch.bfloat16, device=dev)
    do = torch.zeros((1, 0, 2, 64), dtype=torch.float32, device=dev)
    dht = torch.randn((1, 2, 64, 64), device=dev)
    out = axiom_amd.kda_chunk_bwd(q, q, v, q, beta, do, dht=dht)
    torch.cuda.synchronize()
    assert torch.equal(out[5], dht)
    out = axiom_amd.kda_chunk_bwd(q, q, v, q, beta, do)
    torch.cuda.synchronize()
    assert torch.count_nonzero(out[5]) == 0


def test_autograd_function_matches_direct_call(cuda):
    import axiom_amd
    x, do, dS = _case(1, 150, 2, 64, seed=8, prec="fp32")
    ts = {n: to_dev(x[n], torch.float32, cuda).requires_grad_(True) for n in ("q", "k", "v", "g", "beta", "h0")}
    o, ht = axiom_amd.kda_chunk(ts["q"], ts["k"], ts["v"], ts["g"], ts["beta"], initial_state=ts["h0"])
    do_t = to_dev(do, torch.float32, cuda)
    dS_t = to_dev(dS, torch.float32, cuda)
    ((o * do_t).sum() + (ht * dS_t).sum()).backward()
    direct = axiom_amd.kda_chunk_bwd(*(ts[n].detach() for n in ("q", "k", "v", "g", "beta")), do_t,
                                     dht=dS_t, initial_state=ts["h0"].detach())
    torch.cuda.synchronize()
    for n, dref in zip(("q", "k", "v", "g", "beta", "h0"), direct):
        assert torch.equal(ts[n].grad, dref), n


def test_bwd_long_chain_bf16(cuda):
    """1 024 tokens (16 chunks per chain), d = 128: the scans carry across many chunks."""
    x, do, dS = _case(1, 1024, 2, 128, seed=12, prec="bf16")
    got = _hip(cuda, x, do, dS, "bf16")
    _check_all(got, x, do, dS, 1.0, "bf16")
