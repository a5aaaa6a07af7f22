"""kda_chunk_fwd_noalloc (the forward with the library's per-device scratch
in place of a caller workspace) against kda_chunk_fwd, through the C ABI.

Both entry points run the same kernels on the same workspace layout, so the
results must agree bit for bit.  Two calls in a row on the shared scratch,
the second smaller and of another dtype (so the second reads nothing the
first left behind), and a call whose workspace exceeds the scratch, which
must be refused before anything is enqueued.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle import inputs
from tests.kda_testutil import TDT, to_dev

pytestmark = pytest.mark.gpu


def _args(cuda, B, T, H, d, prec, seed, h0_std):
    x = inputs.make_inputs(B, T, H, d, d, seed=seed, dtype="bf16" if prec == "bf16" else "fp32",
                           h0_std=h0_std)
    dt = TDT[prec]
    t = {n: to_dev(x[n], dt, cuda) for n in ("q", "k", "v", "g", "beta")}
    t["h0"] = to_dev(x["h0"], torch.float32, cuda) if h0_std > 0 else None
    return t


def _call(cuda, t, B, T, H, d, in_code, noalloc):
    from axiom_amd import _lib
    L = _lib.lib()
    p = lambda a: ctypes.c_void_p(0 if a is None else a.data_ptr())  # noqa: E731
    o = torch.full((B, T, H, d), float("nan"), dtype=torch.float32, device=cuda)
    ht = torch.full((B, H, d, d), float("nan"), dtype=torch.float32, device=cuda)
    stream = ctypes.c_void_p(torch.cuda.current_stream(cuda).cuda_stream)
    common = (stream, p(t["q"]), p(t["k"]), p(t["v"]), p(t["g"]), p(t["beta"]), p(t["h0"]),
              ctypes.c_void_p(0), 0, p(o), p(ht), B, T, H, d, d, 64, 1.0, in_code, _lib.KDA_DTYPE_F32)
    if noalloc:
        rc = L.kda_chunk_fwd_noalloc(*common)
    else:
        nb = L.kda_chunk_fwd_workspace(B, T, H, d, d, 64, 0, in_code)
        ws = torch.empty(nb, dtype=torch.uint8, device=cuda)
        rc = L.kda_chunk_fwd(*common, p(ws), nb)
    torch.cuda.synchronize()
    assert rc == _lib.KDA_OK, _lib.last_error()
    return o, ht


@pytest.mark.parametrize("first,second", [
    ((4, 4096, 16, 128, "bf16", 1, 0.02), (1, 200, 2, 64, "fp32", 2, 0.05)),
    ((2, 1500, 8, 128, "bf16", 3, 0.0), (1, 70, 3, 128, "fp16", 4, 0.02)),
])
def test_noalloc_equals_workspace_entry(cuda, first, second):
    from axiom_amd import _lib
    codes = {"bf16": _lib.KDA_DTYPE_BF16, "fp16": _lib.KDA_DTYPE_F16, "fp32": _lib.KDA_DTYPE_F32}
    for B, T, H, d, prec, seed, h0 in (first, second):
        print(f"[noalloc] B={B} T={T} H={H} d={d} {prec}", flush=True)
        t = _args(cuda, B, T, H, d, prec, seed, h0)
        o_ref, ht_ref = _call(cuda, t, B, T, H, d, codes[prec], noalloc=False)
        o, ht = _call(cuda, t, B, T, H, d, codes[prec], noalloc=True)
        assert torch.isfinite(o_ref).all() and torch.isfinite(ht_ref).all()
        assert torch.equal(o, o_ref) and torch.equal(ht, ht_ref)


def test_noalloc_refuses_a_call_beyond_its_scratch(cuda):
    """A varlen call of 64 sequences over T = 300 000 tokens needs ~5.8 GB of
    workspace: refused with KDA_ERR_WORKSPACE naming the scratch size."""
    from axiom_amd import _lib
    L = _lib.lib()
    t = _args(cuda, 1, 64, 2, 128, "bf16", 5, 0.0)
    cu = torch.zeros(65, dtype=torch.int32, device=cuda)
    o = torch.empty(1, 64, 2, 128, device=cuda)
    p = lambda a: ctypes.c_void_p(a.data_ptr())  # noqa: E731
    stream = ctypes.c_void_p(torch.cuda.current_stream(cuda).cuda_stream)
    rc = L.kda_chunk_fwd_noalloc(stream, p(t["q"]), p(t["k"]), p(t["v"]), p(t["g"]), p(t["beta"]),
                                 ctypes.c_void_p(0), p(cu), 64, p(o), ctypes.c_void_p(0),
                                 1, 300000, 16, 128, 128, 64, 1.0, _lib.KDA_DTYPE_BF16, _lib.KDA_DTYPE_F32)
    torch.cuda.synchronize()
    assert rc == _lib.KDA_ERR_WORKSPACE
    msg = _lib.last_error()
    assert "scratch" in msg and "201326592" in msg, msg
