"""Shared helpers of the KDA tests: input transfer and the parity bars."""

from __future__ import annotations

import numpy as np
import torch

from oracle import kda_oracle as K

# Parity bars: relative L2 and max-abs error of o
# and of the final state against the fp64 oracle on identical inputs.
TOL = {
    "bf16": (1e-3, 2e-2),
    "fp16": (1e-3, 2e-2),
    "fp32": (1e-5, 1e-5),
}

TDT = {"bf16": torch.bfloat16, "fp16": torch.float16, "fp32": torch.float32}


def to_dev(x: np.ndarray, dtype, device):
    return torch.from_numpy(np.ascontiguousarray(x)).to(device=device, dtype=dtype)


def assert_close(name: str, got, ref, tol: tuple[float, float]):
    got = got.detach().float().cpu().numpy() if isinstance(got, torch.Tensor) else np.asarray(got)
    ref = ref.detach().cpu().numpy() if isinstance(ref, torch.Tensor) else np.asarray(ref)
    assert got.shape == ref.shape, f"{name}: shape {got.shape} vs {ref.shape}"
    assert np.all(np.isfinite(got)), f"{name}: non-finite values"
    rel = K.rel_l2(got, ref)
    mx = K.max_abs(got, ref)
    rel_tol, abs_tol = tol
    assert rel <= rel_tol and mx <= abs_tol, (
        f"{name}: rel_l2={rel:.3e} (tol {rel_tol:g}) max_abs={mx:.3e} (tol {abs_tol:g})")
    return rel, mx


def make_inputs_device(B, T, H, dk, dv, seed, device, h0_std=0.0, n_states=None):
    """The config distributions drawn on the GPU (torch generator), bf16:
    q, k = l2norm(N(0,1)); v ~ N(0,1); beta = sigmoid(N(0,1));
    g = -softplus(N(0,1)) * exp(a_h), a_h ~ U(-2, 0); h0 ~ N(0, h0_std^2) fp32.
    For full-size cases whose inputs are too large to draw on the host; the
    oracle then sees the exact bf16 values of the chains it checks."""
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)

    def l2n(x):
        return x / (x.norm(dim=-1, keepdim=True) + 1e-12)

    q = l2n(torch.randn(B, T, H, dk, device=device, generator=gen)).to(torch.bfloat16)
    k = l2n(torch.randn(B, T, H, dk, device=device, generator=gen)).to(torch.bfloat16)
    v = torch.randn(B, T, H, dv, device=device, generator=gen).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn(B, T, H, device=device, generator=gen)).to(torch.bfloat16)
    gz = torch.randn(B, T, H, dk, device=device, generator=gen)
    a = torch.rand(H, device=device, generator=gen) * -2.0
    g = (-torch.nn.functional.softplus(gz) * torch.exp(a)[None, None, :, None]).to(torch.bfloat16)
    out = dict(q=q, k=k, v=v, g=g, beta=beta)
    if h0_std > 0.0:
        n = B if n_states is None else n_states
        out["h0"] = torch.randn(n, H, dk, dv, device=device, generator=gen) * h0_std
    return out


def host_chains(d, b, heads, t0=0, t1=None):
    """float32 numpy copies of batch row b, tokens [t0, t1), the given heads."""
    sl = slice(t0, t1)
    res = {}
    for n in ("q", "k", "v", "g"):
        res[n] = d[n][b:b + 1, sl][:, :, heads].float().cpu().numpy()
    res["beta"] = d["beta"][b:b + 1, sl][:, :, heads].float().cpu().numpy()
    return res


def chain_errors(got, ref, chain_axes: tuple[int, ...]):
    """Relative L2 and max-abs error of every chain: the slices at one index
    of ``chain_axes``, reduced over the other axes."""
    got = got.detach().double().cpu().numpy() if isinstance(got, torch.Tensor) else np.asarray(got, np.float64)
    ref = ref.detach().double().cpu().numpy() if isinstance(ref, torch.Tensor) else np.asarray(ref, np.float64)
    assert got.shape == ref.shape, f"shape {got.shape} vs {ref.shape}"
    assert np.all(np.isfinite(got)), "non-finite values"
    red = tuple(i for i in range(got.ndim) if i not in chain_axes)
    err = got - ref
    rel = np.sqrt((err * err).sum(axis=red)) / np.maximum(np.sqrt((ref * ref).sum(axis=red)), 1e-30)
    return rel, np.abs(err).max(axis=red)


def assert_chain_errors(name: str, rel, mx, tol: tuple[float, float]):
    """Every chain's errors (from chain_errors) within ``tol``; returns the worst."""
    rel, mx = np.asarray(rel), np.asarray(mx)
    worst = np.unravel_index(int(np.argmax(rel / tol[0] + mx / tol[1])), rel.shape)
    assert (rel <= tol[0]).all() and (mx <= tol[1]).all(), (
        f"{name}: chain {worst} rel_l2={rel[worst]:.3e} max_abs={mx[worst]:.3e} (tol {tol}); "
        f"{int(((rel > tol[0]) | (mx > tol[1])).sum())} of {rel.size} chains over the bar")
    print(f"  {name}: {rel.size} chains, worst rel_l2={rel.max():.2e} max_abs={mx.max():.2e}", flush=True)
    return float(rel.max()), float(mx.max())


def assert_chains_close(name: str, got, ref, tol: tuple[float, float], chain_axes: tuple[int, ...]):
    """Parity per chain: relative L2 and max-abs error of every chain within
    ``tol``, so that one wrong chain among many cannot hide in a norm over
    all of them.  Returns the worst relative L2 and max-abs over the chains."""
    rel, mx = chain_errors(got, ref, chain_axes)
    return assert_chain_errors(name, rel, mx, tol)
