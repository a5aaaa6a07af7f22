"""Uninitialised-memory probe of every caller-owned buffer.

The entry points take their scratch memory from the caller (a workspace of
the size the matching ``*_workspace`` call reports) and promise that no part
of it needs clearing: every workspace word a call reads is written earlier in
the same call, and every output element is written.  Each case below runs an
entry point twice on the same inputs: once with the workspace and every
output filled with 0xFF bytes (NaN in fp32, bf16 and fp16) and once with them
zeroed.  The results must be bit-identical, and finite.  A read of a stale
word, or an output element left unwritten, shows up as a NaN or as a
difference between the two runs.

Layouts covered: dense calls in one segment, in two sequential segments (the
state carried through the workspace when no final state is asked for) and in
overlapped segments (two alternating result sets); varlen (the prep kernel's
offsets and order in the workspace), also in segments (its position tables,
the state carried through ht or the workspace); exact (fp32) mode; the chunked backward;
the layer forward (fused prologue); the cc_scan seam, its backward rule and
their batched forms.  The reference ran its device checks under a poison
fill of the same kind (evidence/mfu-55/kernels/REPORT-kda-ut-solve.md:20).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from axiom_amd import _lib
from oracle import inputs
from tests.kda_testutil import make_inputs_device

pytestmark = pytest.mark.gpu

_vp = lambda t: None if t is None else t.data_ptr()  # noqa: E731


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _twice(make_bufs, run):
    """run(bufs) with every buffer poisoned, then zeroed: outputs equal bit for bit."""
    res = []
    for fill in (0xFF, 0x00):
        bufs = make_bufs()
        for b in bufs.values():
            if b is not None:
                b.view(torch.uint8).fill_(fill)
        torch.cuda.synchronize()
        outs = run(bufs)
        torch.cuda.synchronize()
        res.append({n: t.clone() for n, t in outs.items()})
    for n in res[0]:
        a, b = res[0][n], res[1][n]
        assert torch.isfinite(b.float()).all(), f"{n}: non-finite with a zeroed workspace"
        assert torch.equal(a.view(torch.uint8), b.view(torch.uint8)), \
            f"{n}: poisoned and zeroed buffers give different results"


def _u8(n, dev):
    return torch.empty(max(int(n), 1), dtype=torch.uint8, device=dev)


def _chunk_fwd_case(cuda, B, T, H, d, dtype, h0, want_ht, cu=None, least=False):
    L = _lib.lib()
    if dtype == "fp32":
        x = inputs.make_inputs(B, T, H, d, d, seed=T + H, dtype="fp32", h0_std=0.05,
                               n_states=None if cu is None else len(cu) - 1)
        ts = {n: torch.from_numpy(x[n]).to(cuda) for n in ("q", "k", "v", "g", "beta")}
        ts["h0"] = torch.from_numpy(x["h0"]).to(cuda)
        code = _lib.KDA_DTYPE_F32
    else:
        ts = make_inputs_device(B, T, H, d, d, seed=T + H, device=cuda, h0_std=0.05,
                                n_states=None if cu is None else len(cu) - 1)
        code = _lib.KDA_DTYPE_BF16
    n_seqs = 0 if cu is None else len(cu) - 1
    N = B if cu is None else n_seqs
    cu_t = None if cu is None else torch.tensor(cu, dtype=torch.int32, device=cuda)
    need = int((L.kda_chunk_fwd_workspace_min if least else L.kda_chunk_fwd_workspace)(B, T, H, d, d, 64, n_seqs, code))
    assert need > 0

    def make_bufs():
        return {"ws": _u8(need, cuda), "o": torch.empty(B, T, H, d, device=cuda),
                "ht": torch.empty(N, H, d, d, device=cuda) if want_ht else None}

    def run(b):
        rc = L.kda_chunk_fwd(_stream(), _vp(ts["q"]), _vp(ts["k"]), _vp(ts["v"]), _vp(ts["g"]), _vp(ts["beta"]),
                             _vp(ts["h0"]) if h0 else None, _vp(cu_t), n_seqs, _vp(b["o"]), _vp(b["ht"]),
                             B, T, H, d, d, 64, 1.0, code, _lib.KDA_DTYPE_F32, _vp(b["ws"]), need)
        _lib.check(rc, "kda_chunk_fwd")
        return {"o": b["o"]} | ({"ht": b["ht"]} if want_ht else {})

    _twice(make_bufs, run)


@pytest.mark.parametrize("B,T,H,d,dtype,h0,want_ht", [
    (1, 200, 2, 128, "bf16", True, True),      # one segment, ragged tail
    (1, 2048, 2, 128, "bf16", True, True),     # two overlapped segments (two result sets)
    (1, 2100, 3, 64, "bf16", False, False),    # overlapped, no h0, no final state
    (4, 4096, 16, 128, "bf16", False, True),   # config 1: two sequential segments
    (4, 4096, 16, 128, "bf16", True, False),   # the same, state carried in the workspace
    (2, 130, 2, 64, "fp32", True, True),       # exact mode
])
def test_chunk_fwd_poisoned_workspace(cuda, B, T, H, d, dtype, h0, want_ht):
    print(f"[poison chunk_fwd] B={B} T={T} H={H} d={d} {dtype} h0={h0} ht={want_ht}", flush=True)
    _chunk_fwd_case(cuda, B, T, H, d, dtype, h0, want_ht)


@pytest.mark.parametrize("lengths,H,d,want_ht", [
    ([100, 1, 0, 640, 77, 300], 2, 128, True),
    ([64, 129, 5], 2, 64, True),
    ([900, 0, 1, 640, 130, 2000, 64, 65], 128, 64, True),    # least workspace, segmented: state in ht
    ([900, 0, 1, 640, 130, 2000, 64, 65], 128, 64, False),   # segmented: state carried in the workspace
])
def test_chunk_fwd_varlen_poisoned_workspace(cuda, lengths, H, d, want_ht):
    cu = [0] + list(np.cumsum(lengths))
    print(f"[poison varlen] lengths={lengths} H={H} d={d} ht={want_ht}", flush=True)
    _chunk_fwd_case(cuda, 1, int(cu[-1]), H, d, "bf16", True, want_ht, cu=cu, least=H > 2)


@pytest.mark.parametrize("B,T,H,d", [(1, 200, 2, 128), (2, 130, 2, 64)])
def test_chunk_bwd_poisoned_workspace(cuda, B, T, H, d):
    L = _lib.lib()
    ts = make_inputs_device(B, T, H, d, d, seed=5, device=cuda, h0_std=0.05)
    gen = torch.Generator(device=cuda)
    gen.manual_seed(9)
    do = torch.randn(B, T, H, d, device=cuda, generator=gen)
    dht = torch.randn(B, H, d, d, device=cuda, generator=gen) * 0.1
    need = int(L.kda_chunk_bwd_workspace(B, T, H, d, d, 64))
    names = ("dq", "dk", "dv", "dg", "dbeta", "dh0")
    shapes = ((B, T, H, d),) * 4 + ((B, T, H), (B, H, d, d))

    def make_bufs():
        return {"ws": _u8(need, cuda)} | {n: torch.empty(s, device=cuda) for n, s in zip(names, shapes)}

    def run(b):
        print(f"[poison chunk_bwd] B={B} T={T} H={H} d={d}", flush=True)
        rc = L.kda_chunk_bwd(_stream(), *(_vp(ts[n]) for n in ("q", "k", "v", "g", "beta")), _vp(ts["h0"]),
                             _vp(do), _vp(dht), *(_vp(b[n]) for n in names), B, T, H, d, d, 64, 1.0,
                             _lib.KDA_DTYPE_BF16, _lib.KDA_DTYPE_F32, _vp(b["ws"]), need)
        _lib.check(rc, "kda_chunk_bwd")
        return {n: b[n] for n in names}

    _twice(make_bufs, run)


@pytest.mark.parametrize("B,T,H,d,K", [(2, 200, 2, 128, 4), (1, 100, 2, 64, 6)])
def test_layer_fwd_poisoned_workspace(cuda, B, T, H, d, K):
    L = _lib.lib()
    gen = torch.Generator(device=cuda)
    gen.manual_seed(3)
    HD = H * d
    xs = [torch.randn(B, T, HD, device=cuda, generator=gen).to(torch.bfloat16) for _ in range(3)]
    ws_ = [torch.randn(K, HD, device=cuda, generator=gen) * 0.4 for _ in range(3)]
    bin_ = [torch.randn(B, K - 1, HD, device=cuda, generator=gen) for _ in range(3)]
    base = make_inputs_device(B, T, H, d, d, seed=4, device=cuda, h0_std=0.05)
    gate = torch.randn(B, T, HD, device=cuda, generator=gen).to(torch.bfloat16)
    code = _lib.KDA_DTYPE_BF16
    need = int(L.kda_layer_fwd_workspace(B, T, H, d, K, code))

    def make_bufs():
        b = {"ws": _u8(need, cuda), "y": torch.empty(B, T, HD, device=cuda), "ht": torch.empty(B, H, d, d, device=cuda),
             "o": torch.empty(B, T, H, d, device=cuda)}
        for i in range(3):
            b[f"b{i}"] = torch.empty(B, K - 1, HD, device=cuda)
        return b

    def run(b):
        print(f"[poison layer_fwd] B={B} T={T} H={H} d={d} K={K}", flush=True)
        rc = L.kda_layer_fwd(_stream(), *(_vp(x) for x in xs), _vp(base["g"]), _vp(base["beta"]), _vp(gate),
                             *(_vp(w) for w in ws_), *(_vp(x) for x in bin_), *(_vp(b[f"b{i}"]) for i in range(3)),
                             _vp(base["h0"]), _vp(b["ht"]), _vp(b["y"]), _vp(b["o"]), B, T, H, d, K, 1.0, 1e-6,
                             code, _lib.KDA_DTYPE_BF16, _lib.KDA_DTYPE_F32, _vp(b["ws"]), need)
        _lib.check(rc, "kda_layer_fwd")
        return {n: b[n] for n in ("y", "ht", "o", "b0", "b1", "b2")}

    _twice(make_bufs, run)


def _seam_inputs(cuda, B, T, H, d, seed):
    gen = torch.Generator(device=cuda)
    gen.manual_seed(seed)
    lead = (B,) if B else ()
    n = lambda *s: torch.randn(*lead, *s, device=cuda, generator=gen)  # noqa: E731
    l2 = lambda x: x / x.norm(dim=-1, keepdim=True)  # noqa: E731
    q = l2(n(T, H, d)).reshape(*lead, T, H * d).to(torch.bfloat16)
    k = l2(n(T, H, d)).reshape(*lead, T, H * d).to(torch.bfloat16)
    v = n(T, H * d).to(torch.bfloat16)
    alpha = torch.exp(-torch.nn.functional.softplus(n(T, H * d)) * 0.3)
    beta32 = torch.sigmoid(n(T, H, 1)).expand(*lead, T, H, 32).reshape(*lead, T, H * 32).contiguous()
    S = n(H, d, d) * 0.05
    do = n(T, H * d)
    dS = n(H, d, d) * 0.1
    return q, k, v, alpha, beta32, S, do, dS


@pytest.mark.parametrize("B,T,H,d", [(0, 4096, 2, 128), (0, 192, 3, 64), (3, 512, 2, 128)])
def test_cc_scan_poisoned_workspace(cuda, B, T, H, d):
    """cc_scan (B = 0: the unbatched entry) or kda_cc_scan_batched, forward and backward rule."""
    L = _lib.lib()
    q, k, v, alpha, beta32, S, do, dS = _seam_inputs(cuda, B, T, H, d, seed=T + d)
    lead = (B,) if B else ()
    need_f = int(L.kda_cc_scan_batched_workspace(B, T, H, d, d, 64) if B else L.kda_cc_scan_workspace(T, H, d, d, 64))
    need_b = int(L.kda_cc_scan_bwd_batched_workspace(B, T, H, d, d, 64) if B
                 else L.kda_cc_scan_bwd_workspace(T, H, d, d, 64))

    def make_f():
        return {"ws": _u8(need_f, cuda), "o": torch.empty(*lead, T, H * d, device=cuda),
                "S": torch.empty(*lead, H, d, d, device=cuda)}

    def run_f(b):
        print(f"[poison cc_scan] B={B} T={T} H={H} d={d}", flush=True)
        if B:
            rc = L.kda_cc_scan_batched(_stream(), _vp(q), _vp(k), _vp(v), _vp(alpha), _vp(beta32), _vp(S), _vp(b["o"]),
                                       _vp(b["S"]), B, T, H, d, d, 16, 64, _vp(b["ws"]), need_f)
        else:
            rc = L.kda_cc_scan(_stream(), _vp(q), _vp(k), _vp(v), _vp(alpha), _vp(beta32), _vp(S), _vp(b["o"]),
                               _vp(b["S"]), T, H, d, d, 16, 64, _vp(b["ws"]), need_f)
        _lib.check(rc, "kda_cc_scan")
        return {"o": b["o"], "S": b["S"]}

    _twice(make_f, run_f)

    names = ("dq", "dk", "dv", "dalpha", "dbeta32", "dS_in")
    like = (q, k, v, alpha, beta32, S)

    def make_b():
        return {"ws": _u8(need_b, cuda)} | {n: torch.empty_like(t) for n, t in zip(names, like)}

    def run_b(b):
        print(f"[poison cc_scan_bwd] B={B} T={T} H={H} d={d}", flush=True)
        args = [_vp(t) for t in (q, k, v, alpha, beta32, S, do, dS)] + [_vp(b[n]) for n in names]
        if B:
            rc = L.kda_cc_scan_bwd_batched(_stream(), *args, B, T, H, d, d, 16, 64, _vp(b["ws"]), need_b)
        else:
            rc = L.kda_cc_scan_bwd(_stream(), *args, T, H, d, d, 16, 64, _vp(b["ws"]), need_b)
        _lib.check(rc, "kda_cc_scan_bwd")
        return {n: b[n] for n in names}

    _twice(make_b, run_b)
