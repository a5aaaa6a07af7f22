"""GPU parity of the standalone unit-triangular solve (kda_ut_solve, kda_ut_solve_bwd).

The reference's own contract (net/kernels/kda_ut_solve.py, tests
net/tests/test_kernel_kda_ut_solve.py): a = I + tril(U(-0.25, 0.25), -1)
(H, C, C), b ~ N(0, 1) (H, C, dk + dv) at H=12, C=64, dk=dv=128; the solve
must match an exact triangular solve with no entry outside (atol, rtol) =
(1e-4, 1e-4) for fp32 and (2e-2, 2e-2) for bf16 (:66-88, TOLERANCE), and the
fp32 max-abs error stays below 1e-5; the custom_vjp's (dA, dB) match autograd
of the exact solve within atol 1e-4, rtol 1e-3 (:468-469, :556-571), with dA
exactly zero on and above the diagonal (:574-598).  The exact solve here is
torch.linalg.solve_triangular in float64 on the CPU.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

TOL = {torch.float32: (1e-4, 1e-4), torch.bfloat16: (2e-2, 2e-2)}


def _inputs(H, C, N, seed):
    rng = np.random.default_rng(seed)
    a = np.eye(C, dtype=np.float32) + np.tril(rng.uniform(-0.25, 0.25, (H, C, C)).astype(np.float32), -1)
    b = rng.standard_normal((H, C, N)).astype(np.float32)
    return a, b


def _exact(a64, b64, transpose):
    M = torch.eye(a64.shape[-1], dtype=torch.float64) + torch.tril(a64, -1)
    if transpose:
        return torch.linalg.solve_triangular(M.transpose(1, 2), b64, upper=True, unitriangular=True)
    return torch.linalg.solve_triangular(M, b64, upper=False, unitriangular=True)


def _frac_bad(x, ref, atol, rtol):
    d = (x - ref).abs()
    return float((d > atol + rtol * ref.abs()).double().mean())


@pytest.mark.parametrize("H,C,N", [(12, 64, 256), (3, 17, 100), (2, 64, 1), (1, 1, 5)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("transpose", [False, True])
def test_solve_matches_exact(cuda, H, C, N, dtype, transpose):
    import axiom_amd
    a, b = _inputs(H, C, N, seed=H * 100 + C + N)
    at = torch.from_numpy(a).to(cuda, dtype)
    bt = torch.from_numpy(b).to(cuda, dtype)
    x = axiom_amd.ut_solve(at, bt, transpose=transpose)
    torch.cuda.synchronize()
    assert x.dtype == dtype and x.shape == bt.shape
    ref = _exact(at.double().cpu(), bt.double().cpu(), transpose)
    got = x.double().cpu()
    atol, rtol = TOL[dtype]
    assert _frac_bad(got, ref, atol, rtol) == 0.0, float((got - ref).abs().max())
    if dtype == torch.float32:
        assert float((got - ref).abs().max()) < 1e-5


@pytest.mark.parametrize("transpose", [False, True])
def test_backward_matches_autograd_of_exact_solve(cuda, transpose):
    import axiom_amd
    H, C, N = 12, 64, 256
    a, b = _inputs(H, C, N, seed=7 + transpose)
    dx = np.random.default_rng(3).standard_normal((H, C, N)).astype(np.float32)
    a64 = torch.tensor(a, dtype=torch.float64, requires_grad=True)
    b64 = torch.tensor(b, dtype=torch.float64, requires_grad=True)
    (_exact(a64, b64, transpose) * torch.tensor(dx, dtype=torch.float64)).sum().backward()
    at, bt, dxt = (torch.from_numpy(v).to(cuda) for v in (a, b, dx))
    x = axiom_amd.ut_solve(at, bt, transpose=transpose)
    da, db = axiom_amd.ut_solve_bwd(at, x, dxt, transpose=transpose)
    torch.cuda.synchronize()
    da, db = da.double().cpu(), db.double().cpu()
    mask = torch.tril(torch.ones(C, C, dtype=torch.bool), -1)
    assert torch.allclose(db, b64.grad, atol=1e-4, rtol=1e-3), float((db - b64.grad).abs().max())
    assert torch.allclose(da[:, mask], a64.grad[:, mask], atol=1e-4, rtol=1e-3), \
        float((da[:, mask] - a64.grad[:, mask]).abs().max())
    assert torch.count_nonzero(da[:, ~mask]) == 0


def test_autograd_function_routes_through_the_backward_rule(cuda):
    import axiom_amd
    a, b = _inputs(4, 64, 96, seed=11)
    at = torch.from_numpy(a).to(cuda).requires_grad_(True)
    bt = torch.from_numpy(b).to(cuda).requires_grad_(True)
    dx = torch.randn(4, 64, 96, device=cuda)
    for fn, tr in ((axiom_amd.solve, False), (axiom_amd.solve_t, True)):
        at.grad = bt.grad = None
        x = fn(at, bt)
        (x * dx).sum().backward()
        da, db = axiom_amd.ut_solve_bwd(at.detach(), x.detach(), dx, transpose=tr)
        torch.cuda.synchronize()
        assert torch.equal(at.grad, da) and torch.equal(bt.grad, db)
