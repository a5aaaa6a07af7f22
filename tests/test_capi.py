"""CPU: the C-ABI library loads, exports exactly what ``include/kda_mi355x.h``
declares, and rejects invalid requests before any HIP call.

Nothing here launches a kernel or touches device memory: every call either
only computes sizes or fails argument validation, which the library does on
the host before it enqueues anything.  The Python layer's refusal to run on
CPU tensors (no fallback) is checked too.
"""

from __future__ import annotations

import ctypes
import math
import subprocess

import pytest
import torch

from axiom_amd import _lib
from axiom_amd import kda as kmod

C = 64


@pytest.fixture(scope="module")
def L():
    if not _lib.LIB_PATH.exists():
        from axiom_amd import build
        build.build()
    return _lib.lib()


def _align(x):
    return (x + 255) // 256 * 256


SEGMENT_BUDGET = 160 * 1048576   # bytes of intra-chunk results per segment of a dense call


INTRA_SLOTS = 512   # intra workgroups resident at once: segments are rounded up to whole rounds

# Calls whose 32-column state grid is at most 96 workgroups overlap each
# segment's state scan with the next segment's intra work: two sets of intra
# results, 96 MiB segments, no rounding to whole intra rounds.
OVERLAP_BUDGET = 96 * 1048576
OVERLAP_MAX_STATE_WGS = 96


def overlap_eligible(B, H, dv, es):
    return es == 2 and -(-(B * H) // 8) * 8 * (dv // 32) <= OVERLAP_MAX_STATE_WGS


def dense_segments(B, T, H, dk, dv, es):
    NT = (T + C - 1) // C
    if NT <= 1:
        return 1, NT
    total = B * NT * H * (C * (3 * dk + dv + C) * es + dk * 4)
    ovl = overlap_eligible(B, H, dv, es)
    s = -(-total // (OVERLAP_BUDGET if ovl else SEGMENT_BUDGET))
    if ovl and s < 2 and NT >= 32:
        s = 2   # an overlapped call of 32 or more chunks runs at least two segments
    s = min(max(s, 1), NT)
    seg = -(-NT // s)
    if s > 1 and not ovl:
        m = INTRA_SLOTS // math.gcd(INTRA_SLOTS, B * H)
        up = -(-seg // m) * m
        if up < NT:
            seg = up
    return -(-NT // seg), seg


def dense_ws_bytes(B, T, H, dk, dv, es):
    """Dense workspace size: W, gamma*q, lambda*k [units*H][C][dk], U [..][C][dv],
    Aqk [..][C][C] in operand precision, gamma_C [..][dk] fp32, each 256-B aligned,
    for one segment's units (two sets when segments overlap); plus the carried
    state when the call is segmented."""
    segments, seg = dense_segments(B, T, H, dk, dv, es)
    ch = B * seg * H
    bufs = 2 if (segments > 1 and overlap_eligible(B, H, dv, es)) else 1
    arrays = [bufs * _align(n) for n in (ch * C * dk * es, ch * C * dk * es, ch * C * dk * es, ch * C * dv * es,
                                         ch * C * C * es, ch * dk * 4)]
    if segments > 1:
        arrays.append(B * H * dk * dv * 4)
    arrays.append(4)   # the call's status word
    return sum(_align(n) for n in arrays)


def test_segment_policy():
    # config 1: 304 MB of intra-chunk results -> 2 segments of 32 chunks, each
    # segment's 4 * 16 * 32 = 2048 intra workgroups whole rounds of 512
    assert dense_segments(4, 4096, 16, 128, 128, 2) == (2, 32)
    assert dense_segments(2, 1000, 2, 128, 128, 2) == (1, 16)
    # 70 chunks: 2 segments of 35 chunks rounded up to 40 (whole rounds)
    assert dense_segments(4, 70 * 64, 16, 128, 128, 2) == (2, 40)
    # config 2 (16 chains: 64 state workgroups) overlaps its segments: 96 MiB
    # each, 13 segments of 79 chunks (the last 76)
    assert overlap_eligible(1, 16, 128, 2) and not overlap_eligible(4, 16, 128, 2)
    assert dense_segments(1, 65536, 16, 128, 128, 2) == (13, 79)
    # one segment's worth of results, overlapped: still two segments
    assert dense_segments(1, 4096, 16, 128, 128, 2) == (2, 32)
    assert dense_segments(1, 31 * 64, 16, 128, 128, 2) == (1, 31)
    assert not overlap_eligible(1, 16, 128, 4)   # exact mode never overlaps


VARLEN_BUDGET = 160 * 1048576   # intra-chunk results per segment of a varlen call's least workspace
VARLEN_MAX_SEQS = 2048           # segmented only with the longest-first order


def varlen_min_ku(T, N, H, dk, dv, es):
    """Units per segment of the least workspace, 0 when a call never segments."""
    units = (T + 63 * N) // C   # upper bound on sum(ceil(len_i / C))
    per_unit = H * (C * (3 * dk + dv + C) * es + dk * 4)
    if N <= VARLEN_MAX_SEQS and units * per_unit > VARLEN_BUDGET:
        return max(1, VARLEN_BUDGET // per_unit)
    return 0


def varlen_segments(T, N, H, dk, dv, es):
    """(launches, units per launch) of a varlen call given its least workspace."""
    units = (T + 63 * N) // C
    ku = varlen_min_ku(T, N, H, dk, dv, es)
    return (-(-units // ku), ku) if ku else (1, units)


def varlen_ws_bytes(T, N, H, dk, dv, es, ku=0):
    """Varlen workspace: the intra-chunk results of one launch's units, the
    prep kernel's tables (cu_clamped, chunk offsets, unit count, order, flags)
    and, when segmented (ku units per launch), the position-major unit tables
    (pos_off over the chunk positions, the segments' first positions) and the
    carried state."""
    units = (T + 63 * N) // C
    segs = -(-units // ku) if 0 < ku < units else 1
    if segs > 1:
        units = ku
    ch = units * H
    arrays = [ch * C * dk * es, ch * C * dk * es, ch * C * dk * es, ch * C * dv * es,
              ch * C * C * es, ch * dk * 4, (N + 1) * 4, (N + 1) * 4, 4, N * 4, 4]
    if segs > 1:
        arrays += [((T + C - 1) // C + 2) * 4, (segs + 1) * 2 * 4, N * H * dk * dv * 4]
    arrays.append(4)   # the call's status word
    return sum(_align(n) for n in arrays)


def test_varlen_segment_policy():
    # config 3 (64 sequences, T = 309 178, H 16 d 128): 4 894 units at most;
    # its least workspace runs segments of 141 units (160 MiB of results), 35 launches
    assert varlen_segments(309178, 64, 16, 128, 128, 2) == (35, 141)
    assert varlen_segments(108, 4, 16, 128, 128, 2) == (1, 5)
    assert varlen_segments(10 ** 6, 3000, 16, 128, 128, 2)[0] == 1   # beyond the sortable count
    assert varlen_ws_bytes(309178, 64, 16, 128, 128, 2, 141) < 240 * 1048576
    assert varlen_ws_bytes(309178, 64, 16, 128, 128, 2) > 5 * 10 ** 9


def test_header_declares_the_abi():
    names = _lib.header_symbols()
    assert set(names) == set(_lib._SIGNATURES), names
    assert len(names) == len(set(names)) == 30


def test_library_exports_every_declared_symbol(L):
    for name in _lib.header_symbols():
        assert hasattr(L, name), f"{name} declared in the header but not exported"
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)],
                         capture_output=True, text=True, check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    kda_exported = {s for s in exported if s.startswith("kda_")}
    assert kda_exported == set(_lib.header_symbols()), kda_exported ^ set(_lib.header_symbols())


def test_abi_version(L):
    assert L.kda_abi_version() == 102


@pytest.mark.parametrize("B,T,H,d", [(1, 512, 4, 64), (4, 4096, 16, 128), (2, 1, 3, 128),
                                     (3, 65, 2, 64), (1, 0, 1, 64), (1, 65536, 16, 128),
                                     (1, 100000, 3, 128), (1, 100000, 3, 64), (2, 32768, 16, 128)])
@pytest.mark.parametrize("code,es", [(0, 4), (1, 2), (2, 2), (3, 2)])
def test_dense_workspace_size(L, B, T, H, d, code, es):
    assert L.kda_chunk_fwd_workspace(B, T, H, d, d, C, 0, code) == dense_ws_bytes(B, T, H, d, d, es)


@pytest.mark.parametrize("B,T,H,d", [(4, 4096, 16, 128), (2, 37, 2, 64), (1, 0, 1, 128)])
@pytest.mark.parametrize("K,code,es,fused", [(4, 1, 2, True), (4, 3, 2, True), (1, 1, 2, True),
                                             (5, 1, 2, False), (4, 0, 4, False)])
def test_layer_workspace_size(L, B, T, H, d, K, code, es, fused):
    """chunk workspace + o fp32 (+ q, k, v when the prologue runs as its own pass)."""
    n = B * T * H * d
    want = _align(dense_ws_bytes(B, T, H, d, d, es)) + _align(n * 4)
    if not fused:
        want += 3 * _align(n * es)
    assert L.kda_layer_fwd_workspace(B, T, H, d, K, code) == want


@pytest.mark.parametrize("args", [(1, 64, 1, 96, 4, 1), (1, 64, 1, 64, 0, 1), (1, 64, 1, 64, 9, 1),
                                  (1, 64, 1, 64, 4, 2), (0, 64, 1, 64, 4, 1), (1, -1, 1, 64, 4, 1)])
def test_layer_workspace_rejects_unsupported(L, args):
    assert L.kda_layer_fwd_workspace(*args) == 0


@pytest.mark.parametrize("T,N", [(262144, 64), (309178, 64), (108, 4), (1, 1), (0, 3), (10 ** 6, 3000)])
def test_varlen_workspace_size(L, T, N):
    assert L.kda_chunk_fwd_workspace(1, T, 16, 128, 128, C, N, 1) == varlen_ws_bytes(T, N, 16, 128, 128, 2)
    ku = varlen_min_ku(T, N, 16, 128, 128, 2)
    assert L.kda_chunk_fwd_workspace_min(1, T, 16, 128, 128, C, N, 1) == varlen_ws_bytes(T, N, 16, 128, 128, 2, ku)


@pytest.mark.parametrize("B,T,H,d", [(4, 4096, 16, 128), (1, 65536, 16, 128), (2, 37, 2, 64)])
def test_dense_workspace_min_is_the_workspace(L, B, T, H, d):
    for code in (0, 1, 2, 3):
        assert L.kda_chunk_fwd_workspace_min(B, T, H, d, d, C, 0, code) == \
            L.kda_chunk_fwd_workspace(B, T, H, d, d, C, 0, code)


def test_varlen_workspace_covers_every_split():
    # sum_i ceil(len_i / C) <= (T + (C-1) N) / C for any N lengths summing to T
    import numpy as np
    rng = np.random.default_rng(0)
    for _ in range(200):
        N = int(rng.integers(1, 40))
        lens = rng.integers(0, 300, size=N)
        T = int(lens.sum())
        assert int(np.sum((lens + C - 1) // C)) <= (T + (C - 1) * N) // C


@pytest.mark.parametrize("args", [
    (1, 64, 1, 96, 96, C, 0, 1),     # head dim
    (1, 64, 1, 64, 128, C, 0, 1),    # dk != dv
    (1, 64, 1, 64, 64, 32, 0, 1),    # chunk
    (0, 64, 1, 64, 64, C, 0, 1),     # B
    (1, -1, 1, 64, 64, C, 0, 1),     # T
    (1, 64, 0, 64, 64, C, 0, 1),     # H
    (1, 64, 1, 64, 64, C, 0, 7),     # dtype
])
def test_workspace_size_rejects_unsupported(L, args):
    assert L.kda_chunk_fwd_workspace(*args) == 0


def test_cc_scan_workspace_size(L):
    T, H, d = 512, 4, 64
    adapt = _align(T * H * d * 4) + _align(T * H * 4)
    assert L.kda_cc_scan_workspace(T, H, d, d, 32) == adapt + dense_ws_bytes(1, T, H, d, d, 2)
    assert L.kda_cc_scan_workspace(T, H, 96, 96, 32) == 0


_FAKE = ctypes.c_void_p(0x1000)   # never dereferenced: every call below fails validation
_NULL = ctypes.c_void_p(0)


def _chunk_fwd(L, **kw):
    a = dict(q=_FAKE, k=_FAKE, v=_FAKE, g=_FAKE, beta=_FAKE, h0=_NULL, cu=_NULL, n_seqs=0,
             o=_FAKE, ht=_NULL, B=1, T=64, H=1, dk=64, dv=64, chunk=C, scale=1.0, in_dt=1,
             out_dt=0, ws=_FAKE, ws_bytes=1 << 40)
    a.update(kw)
    rc = L.kda_chunk_fwd(_NULL, a["q"], a["k"], a["v"], a["g"], a["beta"], a["h0"], a["cu"],
                         a["n_seqs"], a["o"], a["ht"], a["B"], a["T"], a["H"], a["dk"], a["dv"],
                         a["chunk"], a["scale"], a["in_dt"], a["out_dt"], a["ws"], a["ws_bytes"])
    return rc, _lib.last_error()


@pytest.mark.parametrize("kw,status,needle", [
    (dict(q=_NULL), _lib.KDA_ERR_INVALID_ARGUMENT, "null input"),
    (dict(o=_NULL), _lib.KDA_ERR_INVALID_ARGUMENT, "null output"),
    (dict(B=0), _lib.KDA_ERR_INVALID_ARGUMENT, "B=0"),
    (dict(T=-5), _lib.KDA_ERR_INVALID_ARGUMENT, "T=-5"),
    (dict(dk=96, dv=96), _lib.KDA_ERR_UNSUPPORTED, "dk=96"),
    (dict(dk=128, dv=64), _lib.KDA_ERR_UNSUPPORTED, "dk=128, dv=64"),
    (dict(chunk=32), _lib.KDA_ERR_UNSUPPORTED, "chunk=32"),
    (dict(in_dt=9), _lib.KDA_ERR_INVALID_ARGUMENT, "in_dtype=9"),
    (dict(out_dt=2), _lib.KDA_ERR_INVALID_ARGUMENT, "out_dtype=2"),
    (dict(scale=float("nan")), _lib.KDA_ERR_INVALID_ARGUMENT, "scale"),
    (dict(cu=_FAKE, n_seqs=2, B=2), _lib.KDA_ERR_INVALID_ARGUMENT, "requires B == 1"),
    (dict(cu=_FAKE, n_seqs=0), _lib.KDA_ERR_INVALID_ARGUMENT, "n_seqs=0"),
    (dict(ws=_NULL), _lib.KDA_ERR_WORKSPACE, "workspace"),
    (dict(ws_bytes=100), _lib.KDA_ERR_WORKSPACE, "too small"),
    (dict(q=ctypes.c_void_p(0x1008)), _lib.KDA_ERR_INVALID_ARGUMENT, "16-byte aligned"),
    (dict(o=ctypes.c_void_p(0x1004)), _lib.KDA_ERR_INVALID_ARGUMENT, "16-byte aligned"),
    (dict(ws=ctypes.c_void_p(0x1002)), _lib.KDA_ERR_INVALID_ARGUMENT, "16-byte aligned"),
])
def test_chunk_fwd_validation(L, kw, status, needle):
    rc, msg = _chunk_fwd(L, **kw)
    assert rc == status, msg
    assert needle in msg, msg


def test_error_message_is_cleared_by_next_call(L):
    rc, msg = _chunk_fwd(L, chunk=32)
    assert rc != 0 and msg
    assert L.kda_chunk_fwd_workspace(1, 64, 1, 64, 64, C, 0, 1) > 0
    rc, msg = _chunk_fwd(L, dk=96, dv=96)
    assert "dk=96" in msg and "chunk" not in msg


def test_recurrent_step_validation(L):
    def call(**kw):
        a = dict(q=_FAKE, state=_FAKE, B=4, H=2, dk=128, dv=128, scale=1.0, in_dt=1, out_dt=0)
        a.update(kw)
        rc = L.kda_recurrent_step(_NULL, a["q"], _FAKE, _FAKE, _FAKE, _FAKE, a["state"], _FAKE,
                                  a["B"], a["H"], a["dk"], a["dv"], a["scale"], a["in_dt"], a["out_dt"])
        return rc, _lib.last_error()
    assert call(state=_NULL)[0] == _lib.KDA_ERR_INVALID_ARGUMENT
    assert call(B=0)[0] == _lib.KDA_ERR_INVALID_ARGUMENT
    assert call(dk=32, dv=32)[0] == _lib.KDA_ERR_UNSUPPORTED
    rc, msg = call(in_dt=3)
    assert rc == _lib.KDA_ERR_INVALID_ARGUMENT and "decode takes" in msg
    assert call(out_dt=2)[0] == _lib.KDA_ERR_INVALID_ARGUMENT
    rc, msg = call(state=ctypes.c_void_p(0x1008))
    assert rc == _lib.KDA_ERR_INVALID_ARGUMENT and "16-byte aligned" in msg


def test_cc_scan_validation_messages(L):
    def call(T=96, H=1, d=64, tile=16, chunk=32, ws_bytes=1 << 40):
        rc = L.kda_cc_scan(_NULL, _FAKE, _FAKE, _FAKE, _FAKE, _FAKE, _FAKE, _FAKE, _FAKE,
                           T, H, d, d, tile, chunk, _FAKE, ws_bytes)
        return rc, _lib.last_error()
    rc, msg = call(T=100)
    assert rc == _lib.KDA_ERR_INVALID_ARGUMENT
    assert msg == "T=100 must be a multiple of the chunk width C=32"   # net/kernels/kda_cc_fused_persist.py:741-742
    assert call(tile=17)[0] == _lib.KDA_ERR_INVALID_ARGUMENT
    assert call(tile=0)[0] == _lib.KDA_ERR_INVALID_ARGUMENT
    assert call(d=96)[0] == _lib.KDA_ERR_UNSUPPORTED
    assert call(ws_bytes=10)[0] == _lib.KDA_ERR_WORKSPACE


def test_python_layer_refuses_cpu_tensors():
    q = torch.zeros(1, 64, 1, 64, dtype=torch.bfloat16)
    beta = torch.zeros(1, 64, 1, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        kmod.kda_chunk_fwd(q, q, q, q, beta)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        kmod.kda_recurrent_step(q[:, 0], q[:, 0], q[:, 0], q[:, 0], beta[:, 0],
                                torch.zeros(1, 1, 64, 64))


def test_python_layer_argument_errors():
    q = torch.zeros(1, 64, 1, 64, dtype=torch.bfloat16)
    beta = torch.zeros(1, 64, 1, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="chunk_size"):
        kmod.kda_chunk_fwd(q, q, q, q, beta, chunk_size=32)
    with pytest.raises(ValueError, match="head dims"):
        q96 = torch.zeros(1, 64, 1, 96, dtype=torch.bfloat16)
        kmod.kda_chunk_fwd(q96, q96, q96, q96, beta)
    with pytest.raises(ValueError, match="requires B == 1"):
        q2 = torch.zeros(2, 64, 1, 64, dtype=torch.bfloat16)
        kmod.kda_chunk_fwd(q2, q2, q2, q2, torch.zeros(2, 64, 1, dtype=torch.bfloat16),
                           cu_seqlens=torch.tensor([0, 64], dtype=torch.int32))
    with pytest.raises(ValueError, match="initial_state"):
        kmod.kda_chunk_fwd(q, q, q, q, beta, initial_state=torch.zeros(1, 1, 64, 32))


def test_cc_scan_reference_errors():
    T, H, d = 100, 1, 64
    q = torch.zeros(T, H * d, dtype=torch.bfloat16)
    a = torch.ones(T, H * d)
    b = torch.ones(T, H * 32)
    S = torch.zeros(H, d, d)
    with pytest.raises(ValueError, match="persistent kernel consumes bf16 q/k/v"):
        kmod.cc_scan(q.float(), q.float(), q.float(), a, b, S)
    with pytest.raises(ValueError, match="T=100 must be a multiple of the chunk width C=32"):
        kmod.cc_scan(q, q, q, a, b, S)


@pytest.mark.parametrize("args,status,needle", [
    ((_NULL, _FAKE, _FAKE, 1, 64, 8, 0, 0), _lib.KDA_ERR_INVALID_ARGUMENT, "null"),
    ((_FAKE, _FAKE, _FAKE, 1, 65, 8, 0, 0), _lib.KDA_ERR_UNSUPPORTED, "C=65"),
    ((_FAKE, _FAKE, _FAKE, 1, 0, 8, 0, 0), _lib.KDA_ERR_UNSUPPORTED, "C=0"),
    ((_FAKE, _FAKE, _FAKE, 0, 64, 8, 0, 0), _lib.KDA_ERR_INVALID_ARGUMENT, "H=0"),
    ((_FAKE, _FAKE, _FAKE, 1, 64, 8, 2, 0), _lib.KDA_ERR_INVALID_ARGUMENT, "dtype=2"),
])
def test_ut_solve_validation(L, args, status, needle):
    rc = L.kda_ut_solve(_NULL, *args)
    msg = _lib.last_error()
    assert rc == status and needle in msg, msg


def test_chunk_bwd_workspace_size(L):
    NT = (4096 + 63) // 64
    ch = 4 * NT * 16
    # fp32 arrays gamma q, lambda k, gamma_C, Aqk, T, W, U, S, v~, dS', dv~,
    # then the 16-bit inputs' fragment arrays lambda k, Aqk^T, (gamma q)^T, W^T,
    # W and (lambda k)^T
    expected = sum(_align(n) for n in (ch * 64 * 128 * 4,) * 2 + (ch * 128 * 4, ch * 64 * 64 * 4, ch * 64 * 64 * 4)
                   + (ch * 64 * 128 * 4,) * 2 + (ch * 128 * 128 * 4, ch * 64 * 128 * 4, ch * 128 * 128 * 4,
                                                 ch * 64 * 128 * 4)
                   + (ch * 16 * 1024, ch * 6 * 1024, ch * 16 * 1024, ch * 16 * 1024)
                   + (ch * 16 * 1024, ch * 16 * 1024))
    assert L.kda_chunk_bwd_workspace(4, 4096, 16, 128, 128, C) == expected
    assert L.kda_chunk_bwd_workspace(1, 0, 1, 64, 64, C) > 0
    assert L.kda_chunk_bwd_workspace(1, 64, 1, 96, 96, C) == 0


@pytest.mark.parametrize("B,T,H,d,K", [(4, 4096, 16, 128, 4), (2, 37, 2, 64, 8), (1, 0, 1, 128, 4),
                                       (3, 129, 2, 64, 1)])
def test_prologue_bwd_workspace_size(L, B, T, H, d, K):
    """Per-64-row dw partial sums [3][B][ceil(T/64)][K][H*d] fp32 (256 bytes when
    empty: 0 means unsupported)."""
    hd = H * d
    want = _align(3 * B * ((T + 63) // 64) * K * hd * 4) or 256
    assert L.kda_prologue_bwd_workspace(B, T, H, d, K) == want
    for bad in ((0, T, H, d, K), (B, -1, H, d, K), (B, T, H, 96, K), (B, T, H, d, 0), (B, T, H, d, 9)):
        assert L.kda_prologue_bwd_workspace(*bad) == 0


def test_prologue_bwd_validation(L):
    def call(**kw):
        a = dict(x=_FAKE, w=_FAKE, dy=_FAKE, dx=_FAKE, dw=_FAKE, B=1, T=64, H=1, d=64, K=4, dt=1,
                 ws=_FAKE, ws_bytes=1 << 30)
        a.update(kw)
        rc = L.kda_prologue_bwd(_NULL, a["x"], a["x"], a["x"], a["w"], a["w"], a["w"], _NULL, _NULL, _NULL,
                                a["dy"], a["dy"], a["dy"], a["dx"], a["dx"], a["dx"], a["dw"], a["dw"], a["dw"],
                                _NULL, _NULL, _NULL, a["B"], a["T"], a["H"], a["d"], a["K"], a["dt"],
                                a["ws"], a["ws_bytes"])
        return rc, _lib.last_error()
    assert call(x=_NULL)[0] == _lib.KDA_ERR_INVALID_ARGUMENT
    assert call(dw=_NULL)[0] == _lib.KDA_ERR_INVALID_ARGUMENT
    assert call(d=96)[0] == _lib.KDA_ERR_UNSUPPORTED
    assert call(K=9)[0] == _lib.KDA_ERR_UNSUPPORTED
    assert call(dt=2)[0] == _lib.KDA_ERR_INVALID_ARGUMENT
    rc, msg = call(ws_bytes=16)
    assert rc == _lib.KDA_ERR_WORKSPACE and "too small" in msg


def test_epilogue_bwd_validation(L):
    def call(**kw):
        a = dict(o=_FAKE, dout=_FAKE, B=1, T=8, H=1, dv=64, eps=1e-6, dts=(0, 0, 0, 0))
        a.update(kw)
        rc = L.kda_epilogue_bwd(_NULL, a["o"], _FAKE, _FAKE, a["dout"], _FAKE, a["B"], a["T"], a["H"], a["dv"],
                                a["eps"], *a["dts"])
        return rc, _lib.last_error()
    assert call(o=_NULL)[0] == _lib.KDA_ERR_INVALID_ARGUMENT
    assert call(dout=_NULL)[0] == _lib.KDA_ERR_INVALID_ARGUMENT
    assert call(dv=32)[0] == _lib.KDA_ERR_UNSUPPORTED
    assert call(eps=float("nan"))[0] == _lib.KDA_ERR_INVALID_ARGUMENT
    assert call(dts=(0, 0, 0, 2))[0] == _lib.KDA_ERR_INVALID_ARGUMENT
    assert call(B=0)[0] == _lib.KDA_ERR_INVALID_ARGUMENT


def test_cc_scan_bwd_workspace_and_validation(L):
    T, H, d = 4096, 4, 128
    th = T * H
    want = (_align(th * d * 4) + _align(th * 4) + 4 * _align(th * d * 4) + _align(th * 4)
            + L.kda_chunk_bwd_workspace(1, T, H, d, d, C))
    assert L.kda_cc_scan_bwd_workspace(T, H, d, d, 32) == want
    assert L.kda_cc_scan_bwd_workspace(T, H, 96, 96, 32) == 0

    def call(**kw):
        a = dict(q=_FAKE, do=_FAKE, T=96, H=2, d=128, tile=16, chunk=32, ws=_FAKE, ws_bytes=1 << 30)
        a.update(kw)
        rc = L.kda_cc_scan_bwd(_NULL, a["q"], _FAKE, _FAKE, _FAKE, _FAKE, _FAKE, a["do"], _FAKE,
                               _FAKE, _FAKE, _FAKE, _FAKE, _FAKE, _FAKE, a["T"], a["H"], a["d"], a["d"],
                               a["tile"], a["chunk"], a["ws"], a["ws_bytes"])
        return rc, _lib.last_error()
    assert call(q=_NULL)[0] == _lib.KDA_ERR_INVALID_ARGUMENT
    assert call(do=_NULL)[0] == _lib.KDA_ERR_INVALID_ARGUMENT
    rc, msg = call(chunk=64)
    assert rc == _lib.KDA_ERR_INVALID_ARGUMENT and "multiple of the chunk width" in msg
    assert call(tile=17)[0] == _lib.KDA_ERR_INVALID_ARGUMENT
    assert call(d=96)[0] == _lib.KDA_ERR_UNSUPPORTED
    assert call(ws_bytes=64)[0] == _lib.KDA_ERR_WORKSPACE


_ODD = ctypes.c_void_p(0x1004)   # 4-byte aligned only; never dereferenced


def _args_with(n, odd_at, ints, tail=()):
    ptrs = [_FAKE] * n
    ptrs[odd_at] = _ODD
    return [_NULL] + ptrs + list(ints) + list(tail)


@pytest.mark.parametrize("name,n_ptrs,odd_at,ints,tail", [
    # kda_chunk_bwd: q misaligned (B, T, H, dk, dv, chunk, scale, in_dt, dout_dt, ws, bytes)
    ("kda_chunk_bwd", 14, 0, [1, 64, 1, 64, 64, C, 1.0, 1, 0], [_FAKE, 1 << 40]),
    # kda_cc_scan_bwd_batched: d_o misaligned
    ("kda_cc_scan_bwd_batched", 14, 6, [1, 64, 1, 64, 64, 16, 32], [_FAKE, 1 << 40]),
    # kda_prologue: the fp32 projections (two elements per access) misaligned
    ("kda_prologue", 15, 0, [1, 64, 1, 128, 4, 0, 0], []),
    # kda_epilogue: o (fp32) misaligned
    ("kda_epilogue", 3, 0, [1, 64, 1, 128, 1e-6, 0, 1, 1], []),
    # kda_prologue_bwd: dqp misaligned
    ("kda_prologue_bwd", 21, 12, [1, 64, 1, 128, 4, 1], [_FAKE, 1 << 40]),
    # kda_epilogue_bwd: dout misaligned
    ("kda_epilogue_bwd", 5, 3, [1, 64, 1, 128, 1e-6, 0, 1, 1, 1], []),
    # kda_decode_layer_step: state misaligned
    ("kda_decode_layer_step", 14, 12, [1, 1, 128, 4, 1.0, 1e-6, 1, 1], [_FAKE, 1 << 40]),
    # kda_layer_fwd: g misaligned
    ("kda_layer_fwd", 19, 3, [1, 64, 1, 128, 4, 1.0, 1e-6, 1, 1, 1], [_FAKE, 1 << 40]),
])
def test_misaligned_pointers_are_rejected(L, name, n_ptrs, odd_at, ints, tail):
    """Pointers the kernels access several elements at a time must be aligned to
    that access; a misaligned one is rejected before anything is enqueued."""
    res, argtypes = _lib._SIGNATURES[name]
    args = _args_with(n_ptrs, odd_at, ints, tail)
    assert len(args) == len(argtypes), (name, len(args), len(argtypes))
    rc = getattr(L, name)(*args)
    msg = _lib.last_error()
    assert rc == _lib.KDA_ERR_INVALID_ARGUMENT, msg
    assert "aligned" in msg, msg


def test_cc_scan_rejects_a_misaligned_beta32(L):
    # the intra kernel reads the seam's beta32 rows 16 bytes at a time
    rc = L.kda_cc_scan(_NULL, _FAKE, _FAKE, _FAKE, _FAKE, _ODD, _FAKE, _FAKE, _FAKE,
                       64, 1, 64, 64, 16, 32, _FAKE, 1 << 40)
    msg = _lib.last_error()
    assert rc == _lib.KDA_ERR_INVALID_ARGUMENT and "beta32" in msg and "aligned" in msg, msg
