"""GPU parity of the reference seam's backward rule (``kda_cc_scan_bwd``,
``kernel_bwd`` of ``net/kernels/kda_cc_fused_persist.py:1710``) against the
oracle's ``cc_scan_bwd`` (pinned by finite differences of the seam's forward in
tests/test_oracle_bwd.py), and the differentiable ``cc_scan``.

The HIP backward runs on the bf16 q, k, v the seam takes, with its 16-bit
workspace (fp16 forward-side arrays, tests/test_gpu_bwd.py); the fp32
cotangents (dalpha, dbeta32, dS_in) are held to the chunked backward's bar for
16-bit inputs (relative L2 <= 1e-3, max-abs <= 2e-3 x max(1, max|reference|));
dq, dk, dv come back in the primal dtype, bf16, so their bar adds bf16's
rounding (relative L2 <= 4e-3, max-abs <= 1e-2 x max(1, max|reference|)).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import inputs, kda_oracle as K
from tests.kda_testutil import to_dev

pytestmark = pytest.mark.gpu


def _close(name, got, ref, rel_tol, abs_tol):
    got = got.double().cpu().numpy()
    assert got.shape == ref.shape, (name, got.shape, ref.shape)
    assert np.all(np.isfinite(got)), name
    scale = max(1.0, float(np.abs(ref).max()))
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    err = np.abs(got - ref).max()
    assert rel <= rel_tol and err <= abs_tol * scale, f"{name}: rel_l2={rel:.3e} max_abs={err:.3e} scale={scale:.3g}"


def _seam_case(T, H, d, seed):
    dd = inputs.make_inputs(1, T, H, d, d, seed=seed, dtype="bf16", h0_std=0.05)
    rng = np.random.default_rng(seed + 1)
    alpha = np.exp(dd["g"].astype(np.float64)).astype(np.float32).reshape(T, H * d)
    # unequal columns: the seam's beta is their mean
    beta32 = (np.repeat(dd["beta"][0][..., None], 32, axis=-1)
              + rng.uniform(-0.05, 0.05, (T, H, 32))).astype(np.float32).reshape(T, H * 32)
    do = rng.standard_normal((T, H * d)).astype(np.float32)
    dS = (rng.standard_normal((H, d, d)) * 0.1).astype(np.float32)
    qkv = [dd[n][0].reshape(T, H * d) for n in ("q", "k", "v")]
    return qkv, alpha, beta32, dd["h0"][0], do, dS


def _bf16_values(x):
    return torch.from_numpy(np.ascontiguousarray(x)).bfloat16().double().numpy()


@pytest.mark.parametrize("T,H,d,chunk", [(192, 2, 128, 32), (128, 3, 64, 64), (96, 1, 128, 16)])
def test_cc_scan_bwd_matches_oracle(cuda, T, H, d, chunk):
    import axiom_amd
    qkv, alpha, beta32, S, do, dS = _seam_case(T, H, d, seed=T + d)
    q, k, v = (to_dev(x, torch.bfloat16, cuda) for x in qkv)
    f32 = torch.float32
    out = axiom_amd.cc_scan_bwd(q, k, v, to_dev(alpha, f32, cuda), to_dev(beta32, f32, cuda),
                                to_dev(S, f32, cuda), to_dev(do, f32, cuda), to_dev(dS, f32, cuda),
                                tile=16, chunk=chunk)
    torch.cuda.synchronize()
    assert [t.dtype for t in out] == [torch.bfloat16] * 3 + [f32] * 3
    ref = K.cc_scan_bwd(*(_bf16_values(x) for x in qkv), alpha, beta32, S, do, dS, chunk=64)
    for name, got, r in zip(("dq", "dk", "dv"), out[:3], ref[:3]):
        _close(name, got, r, 4e-3, 1e-2)
    for name, got, r in zip(("dalpha", "dbeta32", "dS_in"), out[3:], ref[3:]):
        _close(name, got, r, 1e-3, 2e-3)


def test_cc_scan_autograd_equals_the_backward_rule(cuda):
    """``cc_scan`` under torch autograd hands back exactly ``cc_scan_bwd``'s
    cotangents (the custom_vjp contract), in the primal dtypes."""
    import axiom_amd
    T, H, d = 128, 2, 128
    qkv, alpha, beta32, S, do, dS = _seam_case(T, H, d, seed=7)
    f32 = torch.float32
    leaves = [to_dev(x, torch.bfloat16, cuda) for x in qkv] + \
             [to_dev(alpha, f32, cuda), to_dev(beta32, f32, cuda), to_dev(S, f32, cuda)]
    for t in leaves:
        t.requires_grad_(True)
    o, S_new = axiom_amd.cc_scan(*leaves, tile=16, chunk=32)
    do_t, dS_t = to_dev(do, f32, cuda), to_dev(dS, f32, cuda)
    ((o * do_t).sum() + (S_new * dS_t).sum()).backward()
    torch.cuda.synchronize()
    want = axiom_amd.cc_scan_bwd(*(t.detach() for t in leaves), do_t, dS_t, tile=16, chunk=32)
    torch.cuda.synchronize()
    for t, w in zip(leaves, want):
        assert t.grad.dtype == t.dtype
        assert torch.equal(t.grad, w)


def test_cc_scan_bwd_errors(cuda):
    import axiom_amd
    T, H, d = 96, 2, 128
    z = torch.zeros((T, H * d), device=cuda)
    b32 = torch.zeros((T, H * 32), device=cuda)
    S = torch.zeros((H, d, d), device=cuda)
    with pytest.raises(ValueError, match="multiple of the chunk width"):
        axiom_amd.cc_scan_bwd(z.bfloat16(), z.bfloat16(), z.bfloat16(), z, b32, S, z, chunk=64)
    with pytest.raises(ValueError, match="persistent backward kernel consumes bf16"):
        axiom_amd.cc_scan_bwd(z, z, z, z, b32, S, z, chunk=32)


def _seam_device(cuda, B, T, H, d, seed):
    """Seam operands at full size drawn on the GPU (config-1 distributions;
    beta32's columns unequal), with a leading batch axis when B > 0."""
    gen = torch.Generator(device=cuda)
    gen.manual_seed(seed)
    lead = (B,) if B else ()
    n = lambda *s: torch.randn(*lead, *s, device=cuda, generator=gen)  # noqa: E731
    l2 = lambda x: x / (x.norm(dim=-1, keepdim=True) + 1e-12)  # noqa: E731
    q = l2(n(T, H, d)).reshape(*lead, T, H * d).to(torch.bfloat16)
    k = l2(n(T, H, d)).reshape(*lead, T, H * d).to(torch.bfloat16)
    v = n(T, H * d).to(torch.bfloat16)
    a = torch.rand(H, device=cuda, generator=gen) * -2.0
    g = -torch.nn.functional.softplus(n(T, H, d)) * torch.exp(a)[:, None]
    alpha = torch.exp(g).reshape(*lead, T, H * d)
    beta32 = (torch.sigmoid(n(T, H, 1)) + (torch.rand(*lead, T, H, 32, device=cuda, generator=gen) - 0.5) * 0.1)
    beta32 = beta32.reshape(*lead, T, H * 32).contiguous()
    S = n(H, d, d) * 0.05
    do = n(T, H * d)
    dS = n(H, d, d) * 0.1
    return q, k, v, alpha, beta32, S, do, dS


def _check_heads(tag, got, ref_fn, heads, H, d):
    """Each sampled head (chain) of one batch element against the oracle on
    that head's operands alone (heads are independent chains)."""
    cols = np.concatenate([np.arange(h * d, (h + 1) * d) for h in heads])
    cols32 = np.concatenate([np.arange(h * 32, (h + 1) * 32) for h in heads])
    ref = ref_fn(cols, cols32)
    T = got[0].shape[0]
    n = len(heads)
    for name, g, r, width, rt, at in (("dq", got[0], ref[0], d, 4e-3, 1e-2), ("dk", got[1], ref[1], d, 4e-3, 1e-2),
                                      ("dv", got[2], ref[2], d, 4e-3, 1e-2), ("dalpha", got[3], ref[3], d, 1e-3, 2e-3),
                                      ("dbeta32", got[4], ref[4], 32, 1e-3, 2e-3)):
        gh = g[:, cols if width == d else cols32].double().cpu().numpy().reshape(T, n, width)
        rh = r.reshape(T, n, width)
        for j, h in enumerate(heads):
            _close(f"{tag} {name} head {h}", torch.from_numpy(gh[:, j]), rh[:, j], rt, at)
    gS = got[5][heads].double().cpu().numpy()
    for j, h in enumerate(heads):
        _close(f"{tag} dS_in head {h}", torch.from_numpy(gS[j]), ref[5][j], 1e-3, 2e-3)


def test_cc_scan_bwd_at_the_bench_shape(cuda):
    """The seam's backward rule at the shape bench.py times it at: one batch
    element of config 1 (T4096 H16 d128), every head against the oracle."""
    import axiom_amd
    T, H, d = 4096, 16, 128
    q, k, v, alpha, beta32, S, do, dS = _seam_device(cuda, 0, T, H, d, seed=41)
    print("[seam bwd] T4096 H16 d128", flush=True)
    out = axiom_amd.cc_scan_bwd(q, k, v, alpha, beta32, S, do, dS, tile=16, chunk=64)
    torch.cuda.synchronize()
    host = [t.float().cpu().numpy() for t in (q, k, v, alpha, beta32, S, do, dS)]

    def ref_fn(cols, cols32):
        hs = cols[::d] // d
        return K.cc_scan_bwd(host[0][:, cols], host[1][:, cols], host[2][:, cols], host[3][:, cols],
                             host[4][:, cols32], host[5][hs], host[6][:, cols], host[7][hs], chunk=64)

    _check_heads("seam", out, ref_fn, list(range(H)), H, d)


def test_cc_scan_bwd_batched_at_the_bench_shape(cuda):
    """kda_cc_scan_bwd_batched over the whole of config 1 (B4 T4096 H16 d128)
    in one call, as bench.py times it: four heads of every batch element
    against the oracle, and element 2 equal bit for bit to its own unbatched
    call."""
    import axiom_amd
    B, T, H, d = 4, 4096, 16, 128
    q, k, v, alpha, beta32, S, do, dS = _seam_device(cuda, B, T, H, d, seed=43)
    print("[seam bwd batched] B4 T4096 H16 d128", flush=True)
    out = axiom_amd.cc_scan_bwd(q, k, v, alpha, beta32, S, do, dS, tile=16, chunk=64)
    one = axiom_amd.cc_scan_bwd(*(t[2].contiguous() for t in (q, k, v, alpha, beta32, S, do, dS)), tile=16, chunk=64)
    torch.cuda.synchronize()
    for a, b in zip(out, one):
        assert torch.equal(a[2], b)
    for b in range(B):
        host = [t[b].float().cpu().numpy() for t in (q, k, v, alpha, beta32, S, do, dS)]
        heads = [(5 * b + 3 * j) % H for j in range(4)]

        def ref_fn(cols, cols32, host=host):
            hs = cols[::d] // d
            return K.cc_scan_bwd(host[0][:, cols], host[1][:, cols], host[2][:, cols], host[3][:, cols],
                                 host[4][:, cols32], host[5][hs], host[6][:, cols], host[7][hs], chunk=64)

        _check_heads(f"batched b={b}", [t[b] for t in out], ref_fn, heads, H, d)
