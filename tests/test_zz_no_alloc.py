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
    """A varlen call of 3 000 sequences over T = 300 000 tokens (more than the
    2 048 the segmented schedule sorts, so its least workspace is the ~6 GB
    of running every chunk-head at once): refused with KDA_ERR_WORKSPACE
    naming the scratch size, before anything is enqueued."""
    from axiom_amd import _lib
    L = _lib.lib()
    t = _args(cuda, 1, 64, 2, 128, "bf16", 5, 0.0)
    cu = torch.zeros(3001, dtype=torch.int32, device=cuda)
    o = torch.empty(1, 64, 2, 128, device=cuda)
    p = lambda a: ctypes.c_void_p(a.data_ptr())  # noqa: E731
    stream = ctypes.c_void_p(torch.cuda.current_stream(cuda).cuda_stream)
    assert L.kda_chunk_fwd_workspace_min(1, 300000, 16, 128, 128, 64, 3000, _lib.KDA_DTYPE_BF16) > 256 << 20
    rc = L.kda_chunk_fwd_noalloc(stream, p(t["q"]), p(t["k"]), p(t["v"]), p(t["g"]), p(t["beta"]),
                                 ctypes.c_void_p(0), p(cu), 3000, p(o), ctypes.c_void_p(0),
                                 1, 300000, 16, 128, 128, 64, 1.0, _lib.KDA_DTYPE_BF16, _lib.KDA_DTYPE_F32)
    torch.cuda.synchronize()
    assert rc == _lib.KDA_ERR_WORKSPACE
    msg = _lib.last_error()
    assert "scratch" in msg and "268435456" in msg, msg


def test_noalloc_runs_config3_in_segments(cuda):
    """Config 3 (64 packed sequences, T = 309 178, H 16 d 128, per-sequence
    h0): its fastest schedule needs ~5.8 GB, so the allocation-free call runs
    the varlen segments that fit the 256 MiB scratch; o and the final states
    equal kda_chunk_fwd's with the full workspace bit for bit, twice in a
    row (the second call over the first's scratch contents), and a smaller
    varlen call after it as well."""
    from axiom_amd import _lib
    from oracle import inputs as oin
    from tests.kda_testutil import make_inputs_device
    L = _lib.lib()
    p = lambda a: ctypes.c_void_p(0 if a is None else a.data_ptr())  # noqa: E731
    stream = ctypes.c_void_p(torch.cuda.current_stream(cuda).cuda_stream)
    for n_seq, lo, hi, seed in ((64, 128, 8192, 3), (5, 10, 700, 9)):
        lengths = oin.make_varlen_lengths(n_seq, lo, hi, seed=seed)
        cu = torch.from_numpy(oin.cu_seqlens_from_lengths(lengths)).to(cuda)
        T, H, d = int(lengths.sum()), 16, 128
        x = make_inputs_device(1, T, H, d, d, seed=seed + 100, device=cuda, h0_std=0.02, n_states=n_seq)
        print(f"[noalloc varlen] N={n_seq} T={T}", flush=True)
        outs = []
        for noalloc in (False, True, True):
            o = torch.full((1, T, H, d), float("nan"), device=cuda)
            ht = torch.full((n_seq, H, d, d), float("nan"), device=cuda)
            common = (stream, p(x["q"]), p(x["k"]), p(x["v"]), p(x["g"]), p(x["beta"]), p(x["h0"]), p(cu), n_seq,
                      p(o), p(ht), 1, T, H, d, d, 64, 1.0, _lib.KDA_DTYPE_BF16, _lib.KDA_DTYPE_F32)
            if noalloc:
                rc = L.kda_chunk_fwd_noalloc(*common)
            else:
                nb = L.kda_chunk_fwd_workspace(1, T, H, d, d, 64, n_seq, _lib.KDA_DTYPE_BF16)
                ws = torch.empty(nb, dtype=torch.uint8, device=cuda)
                rc = L.kda_chunk_fwd(*common, p(ws), nb)
            torch.cuda.synchronize()
            assert rc == _lib.KDA_OK, _lib.last_error()
            outs.append((o, ht))
            if not noalloc:
                del ws
        for o, ht in outs[1:]:
            assert torch.equal(o, outs[0][0]) and torch.equal(ht, outs[0][1])
