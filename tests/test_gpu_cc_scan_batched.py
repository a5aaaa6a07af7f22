"""GPU: the seam with a leading batch axis (``kda_cc_scan_batched`` and
``kda_cc_scan_bwd_batched``), the form of the vmapped caller
(``net/model.py:341-347``: ``jax.vmap`` over the batch of ``cc_scan``, whose
``custom_vjp`` rule the reference marks ``vmap_method="expand_dims"``).

Batch elements are independent chains, so the batched call must give, for
every element, exactly what the unbatched call gives on that element: the
kernels see the same per-chain operands and run the same arithmetic, so the
comparison is bit for bit.  One element per case is also checked against the
oracle (``cc_scan`` / ``cc_scan_bwd``) at the unbatched seam's tolerances: the
forward's bf16 bar (relative L2 <= 1e-3, max-abs <= 2e-2), the backward's
(relative L2 <= 4e-3 for the bf16 dq, dk, dv; 1e-3 for the fp32 cotangents).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import inputs, kda_oracle as K
from tests.kda_testutil import TOL, assert_close, to_dev

pytestmark = pytest.mark.gpu

F32 = torch.float32


def _batch_case(B, T, H, d, seed):
    rng = np.random.default_rng(seed)
    dd = inputs.make_inputs(B, T, H, d, d, seed=seed, dtype="bf16", h0_std=0.05)
    alpha = np.exp(dd["g"].astype(np.float64)).astype(np.float32).reshape(B, T, H * d)
    beta32 = (np.repeat(dd["beta"][..., None], 32, axis=-1)
              + rng.uniform(-0.05, 0.05, (B, T, H, 32))).astype(np.float32).reshape(B, T, H * 32)
    qkv = [dd[n].reshape(B, T, H * d) for n in ("q", "k", "v")]
    S = dd["h0"].astype(np.float32)                                   # [B, H, d, d]
    do = rng.standard_normal((B, T, H * d)).astype(np.float32)
    dS = (rng.standard_normal((B, H, d, d)) * 0.1).astype(np.float32)
    return qkv, alpha, beta32, S, do, dS


def _dev(case, cuda):
    qkv, alpha, beta32, S, do, dS = case
    return ([to_dev(x, torch.bfloat16, cuda) for x in qkv] + [to_dev(alpha, F32, cuda), to_dev(beta32, F32, cuda),
            to_dev(S, F32, cuda)], to_dev(do, F32, cuda), to_dev(dS, F32, cuda))


def _bf16_values(x):
    return torch.from_numpy(np.ascontiguousarray(x)).bfloat16().double().numpy()


def _close(name, got, ref, rel_tol, abs_tol):
    got = got.double().cpu().numpy()
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    assert np.all(np.isfinite(got)), name
    scale = max(1.0, float(np.abs(ref).max()))
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    err = np.abs(got - ref).max()
    assert rel <= rel_tol and err <= abs_tol * scale, f"{name}: rel_l2={rel:.3e} max_abs={err:.3e}"


@pytest.mark.parametrize("B,T,H,d,chunk", [(4, 256, 2, 128, 32), (3, 192, 3, 64, 64), (2, 96, 1, 128, 16)])
def test_batched_forward_equals_per_element_calls(cuda, B, T, H, d, chunk):
    import axiom_amd
    case = _batch_case(B, T, H, d, seed=B * 100 + T)
    ops, _, _ = _dev(case, cuda)
    o, S_new = axiom_amd.cc_scan(*ops, tile=16, chunk=chunk)
    torch.cuda.synchronize()
    assert o.shape == (B, T, H * d) and S_new.shape == (B, H, d, d)
    for b in range(B):
        ob, Sb = axiom_amd.cc_scan(*(t[b].contiguous() for t in ops), tile=16, chunk=chunk)
        torch.cuda.synchronize()
        assert torch.equal(o[b], ob), f"o[{b}] differs from its own call"
        assert torch.equal(S_new[b], Sb), f"S_new[{b}] differs from its own call"
    qkv, alpha, beta32, S, _, _ = case
    b = B - 1
    o_ref, S_ref = K.cc_scan(*(_bf16_values(x[b]) for x in qkv), alpha[b], beta32[b], S[b], chunk=64)
    assert_close("o", o[b], o_ref, TOL["bf16"])
    assert_close("S_new", S_new[b], S_ref, TOL["bf16"])


@pytest.mark.parametrize("B,T,H,d,chunk", [(4, 256, 2, 128, 32), (2, 128, 3, 64, 64)])
def test_batched_backward_equals_per_element_calls(cuda, B, T, H, d, chunk):
    import axiom_amd
    case = _batch_case(B, T, H, d, seed=B * 1000 + T + 1)
    ops, do, dS = _dev(case, cuda)
    grads = axiom_amd.cc_scan_bwd(*ops, do, dS, tile=16, chunk=chunk)
    torch.cuda.synchronize()
    for t, g in zip(ops, grads):
        assert g.shape == t.shape and g.dtype == t.dtype
    for b in range(B):
        gb = axiom_amd.cc_scan_bwd(*(t[b].contiguous() for t in ops), do[b].contiguous(), dS[b].contiguous(),
                                   tile=16, chunk=chunk)
        torch.cuda.synchronize()
        for name, g, w in zip(("dq", "dk", "dv", "dalpha", "dbeta32", "dS_in"), grads, gb):
            assert torch.equal(g[b], w), f"{name}[{b}] differs from its own call"
    qkv, alpha, beta32, S, do_h, dS_h = case
    b = 0
    ref = K.cc_scan_bwd(*(_bf16_values(x[b]) for x in qkv), alpha[b], beta32[b], S[b], do_h[b], dS_h[b], chunk=64)
    for name, got, r in zip(("dq", "dk", "dv"), grads[:3], ref[:3]):
        _close(name, got[b], r, 4e-3, 1e-2)
    for name, got, r in zip(("dalpha", "dbeta32", "dS_in"), grads[3:], ref[3:]):
        _close(name, got[b], r, 1e-3, 2e-3)


def test_batched_autograd_equals_the_backward_rule(cuda):
    import axiom_amd
    B, T, H, d = 3, 128, 2, 128
    ops, do, dS = _dev(_batch_case(B, T, H, d, seed=11), cuda)
    for t in ops:
        t.requires_grad_(True)
    o, S_new = axiom_amd.cc_scan(*ops, tile=16, chunk=32)
    ((o * do).sum() + (S_new * dS).sum()).backward()
    torch.cuda.synchronize()
    want = axiom_amd.cc_scan_bwd(*(t.detach() for t in ops), do, dS, tile=16, chunk=32)
    torch.cuda.synchronize()
    for t, w in zip(ops, want):
        assert torch.equal(t.grad, w)


def test_batched_shape_errors(cuda):
    import axiom_amd
    B, T, H, d = 2, 64, 2, 64
    ops, do, _ = _dev(_batch_case(B, T, H, d, seed=5), cuda)
    q, k, v, alpha, beta32, S = ops
    with pytest.raises(ValueError, match=r"S must be \(B, H, dk, dv\)"):
        axiom_amd.cc_scan(q, k, v, alpha, beta32, S[0], chunk=32)
    with pytest.raises(ValueError, match="shapes must be"):
        axiom_amd.cc_scan(q, k, v, alpha, beta32[:1].contiguous(), S, chunk=32)
    with pytest.raises(ValueError, match="do must be"):
        axiom_amd.cc_scan_bwd(q, k, v, alpha, beta32, S, do[0], chunk=32)


@pytest.mark.parametrize("B", [1, 2])
def test_seam_at_the_config1_element_shape(cuda, B):
    """The seam at its production shape, T=4096 H=16 d=128 (one element runs
    as two overlapped segments, two elements as one sequential launch), with
    unequal beta32 columns: sampled heads of every element against the oracle's
    cc_scan on that head alone."""
    import axiom_amd
    T, H, d = 4096, 16, 128
    case = _batch_case(B, T, H, d, seed=4096 + B)
    ops, _, _ = _dev(case, cuda)
    if B == 1:
        o, S_new = axiom_amd.cc_scan(*(t[0].contiguous() for t in ops), tile=16, chunk=64)
        o, S_new = o[None], S_new[None]
    else:
        o, S_new = axiom_amd.cc_scan(*ops, tile=16, chunk=64)
    torch.cuda.synchronize()
    qkv, alpha, beta32, S, _, _ = case
    for b in range(B):
        for h in (0, H - 1):
            cols = slice(h * d, (h + 1) * d)
            o_ref, S_ref = K.cc_scan(*(_bf16_values(x[b][:, cols]) for x in qkv), alpha[b][:, cols],
                                     beta32[b][:, h * 32:(h + 1) * 32], S[b][h:h + 1], chunk=64)
            assert_close(f"o[{b}] head {h}", o[b][:, cols], o_ref, TOL["bf16"])
            assert_close(f"S_new[{b}] head {h}", S_new[b][h:h + 1], S_ref, TOL["bf16"])
