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
