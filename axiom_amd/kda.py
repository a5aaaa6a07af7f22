"""Host-side API of the MI355X KDA path (torch tensors in device memory).

Mirrors the reference's interface for this path (romannekrasovaillm/axiom):

* :func:`cc_scan` -- the whole-sequence KDA scan seam
  ``net/kernels/kda_cc_fused_persist.py:920`` with the same arguments,
  layouts, outputs and error classes (``ValueError`` for dtype / ``T % C`` /
  unsupported configuration, ``RuntimeError`` when no GPU is present, as
  ``net/kda.py:818-822``).
* :func:`kda_chunk_fwd` -- the FLA-style generalisation ``(q, k, v, g, beta,
  initial_state, cu_seqlens) -> (o, final_state)`` of that seam with explicit
  batch, ragged lengths and varlen packing.
* :func:`kda_recurrent_step` -- one decode token, the delta rule of
  ``net/kda.py:298-310`` plus the read-out ``net/kda.py:293``, state in place.
* :func:`kda_chunk_bwd` / :func:`kda_chunk` -- the chunked backward (the
  ``cc_scan`` custom_vjp's backward rule, ``net/kernels/kda_cc_fused_persist.py:1707``)
  and a differentiable ``torch.autograd.Function`` over forward + backward.
* :func:`kda_prologue` / :func:`kda_epilogue` -- short conv, swish and L2 norm
  before the chunked kernels; head-wise RMSNorm and the sigmoid gate after.
* :func:`ut_solve` / :func:`solve` / :func:`solve_t` -- the standalone batched
  unit-triangular solve of ``net/kernels/kda_ut_solve.py`` (both orientations)
  and its custom_vjp.

Every function calls the HIP library through its C ABI on torch's current
stream; nothing here computes on the CPU.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib

_IN_CODES = {torch.float32: _lib.KDA_DTYPE_F32, torch.bfloat16: _lib.KDA_DTYPE_BF16,
             torch.float16: _lib.KDA_DTYPE_F16}
_OUT_CODES = {torch.float32: _lib.KDA_DTYPE_F32, torch.bfloat16: _lib.KDA_DTYPE_BF16}
SUPPORTED_HEAD_DIMS = (64, 128)
CHUNK = 64


def _ptr(t):
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def _stream(device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _require_gpu(tensors, what: str) -> torch.device:
    devs = {t.device for t in tensors if t is not None}
    if len(devs) != 1:
        raise ValueError(f"{what}: all tensors must be on one device, got {sorted(map(str, devs))}")
    dev = devs.pop()
    if dev.type != "cuda" or not torch.cuda.is_available():
        raise RuntimeError(
            f"{what}: the KDA kernels run only on the GPU (HIP, gfx950); got tensors on {dev}. "
            "There is no CPU fallback.")
    return dev


def _contig(name, t):
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _check_dims(dk, dv, what):
    if dk != dv or dk not in SUPPORTED_HEAD_DIMS:
        raise ValueError(f"{what}: head dims dk={dk}, dv={dv} unsupported "
                         f"(this build runs dk == dv in {SUPPORTED_HEAD_DIMS})")


def chunk_fwd_workspace_bytes(B, T, H, dk, dv, n_seqs=0, in_code=_lib.KDA_DTYPE_BF16) -> int:
    """Workspace bytes of the fastest schedule (``kda_chunk_fwd_workspace``)."""
    return int(_lib.lib().kda_chunk_fwd_workspace(B, T, H, dk, dv, CHUNK, n_seqs, in_code))


def chunk_fwd_workspace_min_bytes(B, T, H, dk, dv, n_seqs=0, in_code=_lib.KDA_DTYPE_BF16) -> int:
    """The least workspace a call accepts (``kda_chunk_fwd_workspace_min``):
    a large varlen call given less than the fastest schedule's runs in
    segments that fit it."""
    return int(_lib.lib().kda_chunk_fwd_workspace_min(B, T, H, dk, dv, CHUNK, n_seqs, in_code))


def kda_chunk_fwd(q, k, v, g, beta, initial_state=None, cu_seqlens=None, chunk_size: int = 64,
                  scale: float = 1.0, output_final_state: bool = True,
                  out_dtype=torch.float32, workspace=None, out=None, final_state=None,
                  check_finite: bool = False):
    """Chunked KDA forward; returns ``(o, final_state)`` (``final_state`` None if not requested).

    ``q, k, g [B,T,H,dk]``, ``v [B,T,H,dv]``, ``beta [B,T,H]``; q/k/v share one
    dtype (bf16, fp16 or fp32).  g and beta have the same dtype as q, or fp32
    with bf16 q/k/v.  ``initial_state [N,H,dk,dv]`` fp32 or None (zeros);
    ``cu_seqlens`` int32 ``[N+1]`` on the device (requires B == 1).  fp32
    inputs select the exact (fp32 MFMA) kernels.  ``out`` / ``final_state``:
    optional preallocated outputs (contiguous, the shapes and dtypes returned).
    ``workspace``: an optional uint8 device buffer of at least
    ``chunk_fwd_workspace_min_bytes`` (smaller ones are replaced by a new
    buffer of the fastest schedule's size).
    16-bit inputs run on fp16 matrix-core operands: unit-norm q and k rows
    and |v|, the state and the intermediate U below 2^15 are supported; with
    ``check_finite`` the call synchronises and raises ``ValueError`` when a
    result is not finite (an operand left that range; ``kda_chunk_fwd_status``).
    """
    what = "kda_chunk_fwd"
    if q.dim() != 4 or k.shape != q.shape or g.shape != q.shape:
        raise ValueError(f"{what}: q, k, g must share a [B,T,H,dk] shape")
    B, T, H, dk = q.shape
    if v.dim() != 4 or v.shape[:3] != q.shape[:3]:
        raise ValueError(f"{what}: v must be [B,T,H,dv] matching q")
    dv = v.shape[3]
    if tuple(beta.shape) != (B, T, H):
        raise ValueError(f"{what}: beta must be [B,T,H] = {(B, T, H)}, got {tuple(beta.shape)}")
    if chunk_size != CHUNK:
        raise ValueError(f"{what}: chunk_size={chunk_size} unsupported (this build runs {CHUNK})")
    _check_dims(dk, dv, what)
    if q.dtype not in _IN_CODES or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError(f"{what}: q, k, v must share a dtype in bf16/fp16/fp32")
    if g.dtype == q.dtype and beta.dtype == q.dtype:
        in_code = _IN_CODES[q.dtype]
    elif q.dtype == torch.bfloat16 and g.dtype == torch.float32 and beta.dtype == torch.float32:
        in_code = _lib.KDA_DTYPE_BF16_F32GATES
    else:
        raise ValueError(f"{what}: g/beta dtype must equal q's, or be fp32 with bf16 q/k/v")
    if out_dtype not in _OUT_CODES:
        raise ValueError(f"{what}: out_dtype must be fp32 or bf16")
    n_seqs = 0
    N = B
    if cu_seqlens is not None:
        if cu_seqlens.dtype != torch.int32 or cu_seqlens.dim() != 1 or cu_seqlens.numel() < 2:
            raise ValueError(f"{what}: cu_seqlens must be a 1-D int32 tensor of N+1 >= 2 offsets")
        if B != 1:
            raise ValueError(f"{what}: cu_seqlens requires B == 1, got B={B}")
        n_seqs = cu_seqlens.numel() - 1
        N = n_seqs
    if initial_state is not None:
        if initial_state.dtype != torch.float32 or tuple(initial_state.shape) != (N, H, dk, dv):
            raise ValueError(f"{what}: initial_state must be fp32 [{N},{H},{dk},{dv}]")
    for name, t in (("q", q), ("k", k), ("v", v), ("g", g), ("beta", beta),
                    ("initial_state", initial_state), ("cu_seqlens", cu_seqlens)):
        if t is not None:
            _contig(name, t)
    dev = _require_gpu([q, k, v, g, beta, initial_state, cu_seqlens], what)
    L = _lib.lib()
    ws_bytes = int(L.kda_chunk_fwd_workspace(B, T, H, dk, dv, CHUNK, n_seqs, in_code))
    if ws_bytes == 0:
        raise ValueError(f"{what}: unsupported configuration")
    # a caller workspace of at least the minimum is used as it is (a large
    # varlen call then runs in the segments that fit it); else a new one of
    # the fastest schedule's size
    ws_min = int(L.kda_chunk_fwd_workspace_min(B, T, H, dk, dv, CHUNK, n_seqs, in_code))
    if workspace is not None and workspace.numel() * workspace.element_size() >= ws_min:
        _contig("workspace", workspace)
        ws_bytes = min(ws_bytes, workspace.numel() * workspace.element_size())
    else:
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    if out is not None:
        if tuple(out.shape) != (B, T, H, dv) or out.dtype != out_dtype or out.device != dev:
            raise ValueError(f"{what}: out must be {out_dtype} [{B},{T},{H},{dv}] on {dev}")
        _contig("out", out)
        o = out
    else:
        o = torch.empty((B, T, H, dv), dtype=out_dtype, device=dev)
    if not output_final_state:
        ht = None
    elif final_state is not None:
        if tuple(final_state.shape) != (N, H, dk, dv) or final_state.dtype != torch.float32 \
                or final_state.device != dev:
            raise ValueError(f"{what}: final_state must be fp32 [{N},{H},{dk},{dv}] on {dev}")
        _contig("final_state", final_state)
        ht = final_state
    else:
        ht = torch.empty((N, H, dk, dv), dtype=torch.float32, device=dev)
    rc = L.kda_chunk_fwd(_stream(dev), _ptr(q), _ptr(k), _ptr(v), _ptr(g), _ptr(beta),
                         _ptr(initial_state), _ptr(cu_seqlens), n_seqs, _ptr(o), _ptr(ht),
                         B, T, H, dk, dv, CHUNK, float(scale), in_code, _OUT_CODES[out_dtype],
                         _ptr(workspace), ws_bytes)
    _lib.check(rc, what)
    if check_finite:
        flags = ctypes.c_int32(0)
        rc = L.kda_chunk_fwd_status(_stream(dev), _ptr(workspace), ws_bytes, B, T, H, dk, dv, CHUNK,
                                    n_seqs, in_code, ctypes.byref(flags))
        _lib.check(rc, "kda_chunk_fwd_status")
        if flags.value & _lib.KDA_STATUS_NONFINITE:
            raise ValueError(f"{what}: non-finite result: an fp16 operand left its range (16-bit inputs "
                             "need unit-norm q, k and |v|, |U|, |state| < 2^15; fp32 inputs run exact)")
    return o, ht


def chunk_bwd_workspace_bytes(B, T, H, dk, dv) -> int:
    return int(_lib.lib().kda_chunk_bwd_workspace(B, T, H, dk, dv, CHUNK))


def kda_chunk_bwd(q, k, v, g, beta, do, dht=None, initial_state=None, scale: float = 1.0,
                  chunk_size: int = 64, need_dh0: bool = True, workspace=None):
    """Gradients of ``kda_chunk_fwd`` (dense inputs, no ``cu_seqlens``).

    ``do [B,T,H,dv]`` (fp32 or bf16) and ``dht [B,H,dk,dv]`` fp32 (None = 0)
    are the cotangents of ``o`` and of the final state.  Returns fp32
    ``(dq, dk, dv, dg, dbeta, dh0)`` (``dh0`` None unless ``need_dh0``);
    ``dg`` is the cotangent of the log decay ``g``.  The backward rule of the
    reference's ``cc_scan`` (``net/kernels/kda_cc_fused_persist.py:1707``).
    """
    what = "kda_chunk_bwd"
    if q.dim() != 4 or k.shape != q.shape or g.shape != q.shape:
        raise ValueError(f"{what}: q, k, g must share a [B,T,H,dk] shape")
    B, T, H, dk = q.shape
    if v.dim() != 4 or v.shape[:3] != q.shape[:3]:
        raise ValueError(f"{what}: v must be [B,T,H,dv] matching q")
    dv = v.shape[3]
    if tuple(beta.shape) != (B, T, H):
        raise ValueError(f"{what}: beta must be [B,T,H] = {(B, T, H)}, got {tuple(beta.shape)}")
    if chunk_size != CHUNK:
        raise ValueError(f"{what}: chunk_size={chunk_size} unsupported (this build runs {CHUNK})")
    _check_dims(dk, dv, what)
    if q.dtype not in _IN_CODES or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError(f"{what}: q, k, v must share a dtype in bf16/fp16/fp32")
    if g.dtype == q.dtype and beta.dtype == q.dtype:
        in_code = _IN_CODES[q.dtype]
    elif q.dtype == torch.bfloat16 and g.dtype == torch.float32 and beta.dtype == torch.float32:
        in_code = _lib.KDA_DTYPE_BF16_F32GATES
    else:
        raise ValueError(f"{what}: g/beta dtype must equal q's, or be fp32 with bf16 q/k/v")
    if tuple(do.shape) != (B, T, H, dv) or do.dtype not in _OUT_CODES:
        raise ValueError(f"{what}: do must be fp32 or bf16 [{B},{T},{H},{dv}]")
    for name, st in (("dht", dht), ("initial_state", initial_state)):
        if st is not None and (st.dtype != torch.float32 or tuple(st.shape) != (B, H, dk, dv)):
            raise ValueError(f"{what}: {name} must be fp32 [{B},{H},{dk},{dv}]")
    for name, t in (("q", q), ("k", k), ("v", v), ("g", g), ("beta", beta), ("do", do),
                    ("dht", dht), ("initial_state", initial_state)):
        if t is not None:
            _contig(name, t)
    dev = _require_gpu([q, k, v, g, beta, do, dht, initial_state], what)
    L = _lib.lib()
    ws_bytes = int(L.kda_chunk_bwd_workspace(B, T, H, dk, dv, CHUNK))
    if ws_bytes == 0:
        raise ValueError(f"{what}: unsupported configuration")
    if workspace is None or workspace.numel() * workspace.element_size() < ws_bytes:
        workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    f32 = torch.float32
    dq = torch.empty((B, T, H, dk), dtype=f32, device=dev)
    dk_ = torch.empty((B, T, H, dk), dtype=f32, device=dev)
    dv_ = torch.empty((B, T, H, dv), dtype=f32, device=dev)
    dg = torch.empty((B, T, H, dk), dtype=f32, device=dev)
    dbeta = torch.empty((B, T, H), dtype=f32, device=dev)
    dh0 = torch.empty((B, H, dk, dv), dtype=f32, device=dev) if need_dh0 else None
    rc = L.kda_chunk_bwd(_stream(dev), _ptr(q), _ptr(k), _ptr(v), _ptr(g), _ptr(beta),
                         _ptr(initial_state), _ptr(do), _ptr(dht),
                         _ptr(dq), _ptr(dk_), _ptr(dv_), _ptr(dg), _ptr(dbeta), _ptr(dh0),
                         B, T, H, dk, dv, CHUNK, float(scale), in_code, _OUT_CODES[do.dtype],
                         _ptr(workspace), ws_bytes)
    _lib.check(rc, what)
    return dq, dk_, dv_, dg, dbeta, dh0


class _KDAChunk(torch.autograd.Function):
    """``(o, final_state)`` of the chunked forward with the HIP backward as its VJP."""

    @staticmethod
    def forward(ctx, q, k, v, g, beta, initial_state, scale):
        o, ht = kda_chunk_fwd(q, k, v, g, beta, initial_state=initial_state, scale=scale)
        ctx.save_for_backward(q, k, v, g, beta, initial_state)
        ctx.scale = scale
        return o, ht

    @staticmethod
    def backward(ctx, do, dht):
        q, k, v, g, beta, h0 = ctx.saved_tensors
        if do is None:
            do = torch.zeros(q.shape[:3] + (v.shape[3],), dtype=torch.float32, device=q.device)
        do = do.contiguous()
        if do.dtype not in _OUT_CODES:
            do = do.float()
        dht = None if dht is None else dht.float().contiguous()
        dq, dk, dv, dg, dbeta, dh0 = kda_chunk_bwd(q, k, v, g, beta, do, dht=dht, initial_state=h0,
                                                   scale=ctx.scale, need_dh0=ctx.needs_input_grad[5])
        return (dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype), dg.to(g.dtype), dbeta.to(beta.dtype),
                dh0, None)


def kda_chunk(q, k, v, g, beta, initial_state=None, scale: float = 1.0):
    """Differentiable chunked KDA: ``(o, final_state)`` with the HIP backward.

    Dense ``[B,T,H,d]`` inputs as :func:`kda_chunk_fwd`; gradients flow to q,
    k, v, g, beta and ``initial_state`` (cast back to their dtypes, as the
    reference's ``custom_vjp`` returns primal dtypes).
    """
    return _KDAChunk.apply(q, k, v, g, beta, initial_state, scale)


_UT_CODES = {torch.float32: _lib.KDA_DTYPE_F32, torch.bfloat16: _lib.KDA_DTYPE_BF16}


def _ut_check(a, b, what):
    if a.dim() != 3 or a.shape[1] != a.shape[2]:
        raise ValueError(f"{what}: a must be (H, C, C), got {tuple(a.shape)}")
    H, C = a.shape[0], a.shape[1]
    if b.dim() != 3 or b.shape[0] != H or b.shape[1] != C:
        raise ValueError(f"{what}: b must be (H, C, N) = ({H}, {C}, N), got {tuple(b.shape)}")
    if a.dtype not in _UT_CODES or b.dtype != a.dtype:
        raise ValueError(f"{what}: a and b must share a dtype in fp32/bf16")
    if not 1 <= C <= 64:
        raise ValueError(f"{what}: C={C} unsupported (this build solves 1 <= C <= 64)")
    for name, t in (("a", a), ("b", b)):
        _contig(name, t)
    return H, C, b.shape[2]


def ut_solve(a, b, transpose: bool = False):
    """``X = (I + L)^-1 B`` (``transpose``: ``(I + L)^-T B``), ``L = tril(a, -1)`` per head.

    The reference's ``kernel`` / ``kernel_t`` (``net/kernels/kda_ut_solve.py:525``,
    ``:536``): ``a (H, C, C)`` unit lower triangular, ``b (H, C, N)``, fp32 or
    bf16 (fp32 arithmetic), ``C <= 64``.
    """
    what = "ut_solve"
    H, C, N = _ut_check(a, b, what)
    dev = _require_gpu([a, b], what)
    x = torch.empty_like(b)
    rc = _lib.lib().kda_ut_solve(_stream(dev), _ptr(a), _ptr(b), _ptr(x), H, C, N, _UT_CODES[a.dtype],
                                 1 if transpose else 0)
    _lib.check(rc, what)
    return x


def ut_solve_bwd(a, x, dx, transpose: bool = False):
    """``(dA, dB)`` of :func:`ut_solve` (``net/kernels/kda_ut_solve.py:563`` ``_backward``)."""
    what = "ut_solve_bwd"
    H, C, N = _ut_check(a, dx, what)
    if x.shape != dx.shape or x.dtype != dx.dtype:
        raise ValueError(f"{what}: x and dx must match")
    _contig("x", x)
    dev = _require_gpu([a, x, dx], what)
    da = torch.empty_like(a)
    db = torch.empty_like(dx)
    rc = _lib.lib().kda_ut_solve_bwd(_stream(dev), _ptr(a), _ptr(x), _ptr(dx), _ptr(da), _ptr(db),
                                     H, C, N, _UT_CODES[a.dtype], 1 if transpose else 0)
    _lib.check(rc, what)
    return da, db


class _UTSolve(torch.autograd.Function):
    @staticmethod
    def forward(ctx, a, b, transpose):
        x = ut_solve(a, b, transpose)
        ctx.save_for_backward(a, x)
        ctx.transpose = transpose
        return x

    @staticmethod
    def backward(ctx, dx):
        a, x = ctx.saved_tensors
        da, db = ut_solve_bwd(a, x, dx.contiguous().to(x.dtype), ctx.transpose)
        return da, db, None


def solve(a, b):
    """Differentiable ``(I + L)^-1 B`` (the reference's ``solve``, ``kda_ut_solve.py:628``)."""
    return _UTSolve.apply(a, b, False)


def solve_t(a, b):
    """Differentiable ``(I + L)^-T B`` (the reference's ``solve_t``, ``kda_ut_solve.py:631``)."""
    return _UTSolve.apply(a, b, True)


def kda_prologue(qp, kp, vp, wq, wk, wv, num_heads: int, conv_state=None, return_state: bool = True,
                 out_dtype=torch.bfloat16):
    """Short conv -> swish -> (L2 norm for q, k) of the projections (``net/kda.py:194-202``).

    ``qp, kp, vp [B, T, H*d]`` fp32 or bf16; ``wq, wk, wv [K, H*d]`` fp32 conv
    taps (``w[i]`` weights the input ``i`` steps back); ``conv_state`` None or
    a tuple of three fp32 ``[B, K-1, H*d]`` buffers (the previous ``K-1``
    inputs).  Returns ``(q, k, v [B, T, H, d] in out_dtype, new_state)``
    (``new_state`` None unless ``return_state``); the new buffers may be the
    ones passed in (updated in place) -- a fresh tuple is returned here.
    """
    what = "kda_prologue"
    if qp.dim() != 3 or kp.shape != qp.shape or vp.shape != qp.shape:
        raise ValueError(f"{what}: qp, kp, vp must share a [B,T,H*d] shape")
    B, T, HD = qp.shape
    H = int(num_heads)
    if H < 1 or HD % H:
        raise ValueError(f"{what}: H*d={HD} is not a multiple of num_heads={H}")
    d = HD // H
    if d not in SUPPORTED_HEAD_DIMS:
        raise ValueError(f"{what}: head dim {d} unsupported ({SUPPORTED_HEAD_DIMS})")
    if qp.dtype not in _UT_CODES or kp.dtype != qp.dtype or vp.dtype != qp.dtype or out_dtype not in _UT_CODES:
        raise ValueError(f"{what}: projections and out_dtype must be fp32 or bf16")
    K = wq.shape[0]
    for name, w in (("wq", wq), ("wk", wk), ("wv", wv)):
        if w.dtype != torch.float32 or tuple(w.shape) != (K, HD):
            raise ValueError(f"{what}: {name} must be fp32 [{K},{HD}]")
    if conv_state is not None:
        for st in conv_state:
            if st.dtype != torch.float32 or tuple(st.shape) != (B, K - 1, HD):
                raise ValueError(f"{what}: conv_state buffers must be fp32 [{B},{K - 1},{HD}]")
    tensors = [qp, kp, vp, wq, wk, wv] + list(conv_state or [])
    for i, t in enumerate(tensors):
        _contig(f"arg{i}", t)
    dev = _require_gpu(tensors, what)
    q = torch.empty((B, T, H, d), dtype=out_dtype, device=dev)
    k = torch.empty_like(q)
    v = torch.empty_like(q)
    new = tuple(torch.empty((B, K - 1, HD), dtype=torch.float32, device=dev) for _ in range(3)) \
        if return_state else (None, None, None)
    bin_ = conv_state if conv_state is not None else (None, None, None)
    rc = _lib.lib().kda_prologue(_stream(dev), _ptr(qp), _ptr(kp), _ptr(vp), _ptr(wq), _ptr(wk), _ptr(wv),
                                 *(_ptr(b) for b in bin_), *(_ptr(b) for b in new), _ptr(q), _ptr(k), _ptr(v),
                                 B, T, H, d, K, _UT_CODES[qp.dtype], _UT_CODES[out_dtype])
    _lib.check(rc, what)
    return q, k, v, (new if return_state else None)


def kda_epilogue(o, gate, eps: float = 1e-6, out_dtype=torch.bfloat16):
    """``sigmoid(gate) * headwise_rms_norm(o)`` (``net/kda.py:205-214`` before ``W_o``).

    ``o [B, T, H, dv]``, ``gate [B, T, H*dv]`` logits (fp32 or bf16); returns
    ``[B, T, H*dv]`` in out_dtype.
    """
    what = "kda_epilogue"
    if o.dim() != 4:
        raise ValueError(f"{what}: o must be [B,T,H,dv]")
    B, T, H, dv = o.shape
    if tuple(gate.shape) != (B, T, H * dv):
        raise ValueError(f"{what}: gate must be [{B},{T},{H * dv}]")
    if dv not in SUPPORTED_HEAD_DIMS:
        raise ValueError(f"{what}: dv={dv} unsupported ({SUPPORTED_HEAD_DIMS})")
    if o.dtype not in _UT_CODES or gate.dtype not in _UT_CODES or out_dtype not in _UT_CODES:
        raise ValueError(f"{what}: dtypes must be fp32 or bf16")
    _contig("o", o)
    _contig("gate", gate)
    dev = _require_gpu([o, gate], what)
    y = torch.empty((B, T, H * dv), dtype=out_dtype, device=dev)
    rc = _lib.lib().kda_epilogue(_stream(dev), _ptr(o), _ptr(gate), _ptr(y), B, T, H, dv, float(eps),
                                 _UT_CODES[o.dtype], _UT_CODES[gate.dtype], _UT_CODES[out_dtype])
    _lib.check(rc, what)
    return y


def kda_decode_layer_step(qp, kp, vp, g, beta, gate, wq, wk, wv, conv_state, state, scale: float = 1.0,
                          eps: float = 1e-6, out_dtype=torch.float32, workspace=None):
    """One decode token of the layer (``net/kda.py:277-295`` minus projections and ``W_o``).

    ``qp, kp, vp [B, H*d]``, ``g [B, H, d]``, ``beta [B, H]``, ``gate [B, H*d]``
    (logits) share a dtype (fp32 or bf16); ``wq, wk, wv [K, H*d]`` fp32;
    ``conv_state`` three fp32 ``[B, K-1, H*d]`` buffers and ``state
    [B, H, d, d]`` fp32 are updated in place.  Returns ``y [B, H*d]``.
    """
    what = "kda_decode_layer_step"
    B, H, d = g.shape
    if tuple(qp.shape) != (B, H * d) or kp.shape != qp.shape or vp.shape != qp.shape or gate.shape != qp.shape:
        raise ValueError(f"{what}: qp, kp, vp, gate must be [{B},{H * d}]")
    if tuple(beta.shape) != (B, H) or tuple(state.shape) != (B, H, d, d) or state.dtype != torch.float32:
        raise ValueError(f"{what}: beta [B,H], state fp32 [B,H,d,d] expected")
    dt = qp.dtype
    if dt not in _UT_CODES or any(t.dtype != dt for t in (kp, vp, g, beta, gate)):
        raise ValueError(f"{what}: qp, kp, vp, g, beta, gate must share a dtype in fp32/bf16")
    K = wq.shape[0]
    bq, bk, bv = conv_state
    tensors = [qp, kp, vp, g, beta, gate, wq, wk, wv, bq, bk, bv, state]
    for i, t in enumerate(tensors):
        _contig(f"arg{i}", t)
    dev = _require_gpu(tensors, what)
    L = _lib.lib()
    need = int(L.kda_decode_layer_workspace(B, H, d, _UT_CODES[dt]))
    if need == 0:
        raise ValueError(f"{what}: unsupported configuration")
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    y = torch.empty((B, H * d), dtype=out_dtype, device=dev)
    rc = L.kda_decode_layer_step(_stream(dev), *(_ptr(t) for t in tensors), _ptr(y), B, H, d, K, float(scale),
                                 float(eps), _UT_CODES[dt], _UT_CODES[out_dtype], _ptr(workspace), need)
    _lib.check(rc, what)
    return y


def layer_fwd_workspace_bytes(B, T, H, d, K, in_code=_lib.KDA_DTYPE_BF16) -> int:
    """Workspace bytes :func:`kda_layer_fwd` needs (0 for an unsupported configuration)."""
    return int(_lib.lib().kda_layer_fwd_workspace(B, T, H, d, K, in_code))


def kda_layer_fwd(qp, kp, vp, g, beta, gate, wq, wk, wv, conv_state=None, initial_state=None,
                  scale: float = 1.0, eps: float = 1e-6, output_final_state: bool = True,
                  return_conv_state: bool = True, out_dtype=torch.bfloat16, workspace=None, o_out=None):
    """The chunked KDA layer between its projections and ``W_o``.

    ``net/kda.py:790-853`` (short conv -> postprocess -> chunked scan -> output
    gate), with the conv history carried as ``chunk_step`` does
    (``net/kda.py:356-358``).  ``qp, kp, vp [B, T, H*d]`` bf16 (or fp32),
    ``g [B, T, H, d]`` log decay and ``beta [B, T, H]`` in the projections'
    dtype or fp32 (with bf16 projections), ``gate [B, T, H*d]`` logits (fp32
    or bf16), ``wq, wk, wv [K, H*d]`` fp32 conv taps, ``conv_state`` None or
    three fp32 ``[B, K-1, H*d]`` buffers, ``initial_state`` None or fp32
    ``[B, H, d, d]``.  Returns ``(y [B, T, H*d] in out_dtype, final_state or
    None, new_conv_state or None)``.  ``o_out``: None, or a fp32 ``[B, T, H, d]``
    tensor that receives the scan's output o (the epilogue's input).
    """
    what = "kda_layer_fwd"
    if qp.dim() != 3 or kp.shape != qp.shape or vp.shape != qp.shape or gate.shape != qp.shape:
        raise ValueError(f"{what}: qp, kp, vp, gate must share a [B,T,H*d] shape")
    if g.dim() != 4:
        raise ValueError(f"{what}: g must be [B,T,H,d]")
    B, T, H, d = g.shape
    if tuple(qp.shape) != (B, T, H * d) or tuple(beta.shape) != (B, T, H):
        raise ValueError(f"{what}: qp [B,T,H*d], beta [B,T,H] expected for g {tuple(g.shape)}")
    _check_dims(d, d, what)
    if any(t.dtype != qp.dtype for t in (kp, vp)) or beta.dtype != g.dtype:
        raise ValueError(f"{what}: qp, kp, vp share a dtype, and so do g and beta")
    if qp.dtype == torch.bfloat16 and g.dtype == torch.bfloat16:
        code = _lib.KDA_DTYPE_BF16
    elif qp.dtype == torch.bfloat16 and g.dtype == torch.float32:
        code = _lib.KDA_DTYPE_BF16_F32GATES
    elif qp.dtype == torch.float32 and g.dtype == torch.float32:
        code = _lib.KDA_DTYPE_F32
    else:
        raise ValueError(f"{what}: projections bf16 (gates bf16 or fp32) or everything fp32")
    if gate.dtype not in _OUT_CODES or out_dtype not in _OUT_CODES:
        raise ValueError(f"{what}: gate and out_dtype must be fp32 or bf16")
    K = wq.shape[0]
    for name, w in (("wq", wq), ("wk", wk), ("wv", wv)):
        if w.dtype != torch.float32 or tuple(w.shape) != (K, H * d):
            raise ValueError(f"{what}: {name} must be fp32 [{K},{H * d}]")
    if conv_state is not None:
        for st in conv_state:
            if st.dtype != torch.float32 or tuple(st.shape) != (B, K - 1, H * d):
                raise ValueError(f"{what}: conv_state buffers must be fp32 [{B},{K - 1},{H * d}]")
    if initial_state is not None and (initial_state.dtype != torch.float32 or
                                      tuple(initial_state.shape) != (B, H, d, d)):
        raise ValueError(f"{what}: initial_state must be fp32 [{B},{H},{d},{d}]")
    if o_out is not None and (o_out.dtype != torch.float32 or tuple(o_out.shape) != (B, T, H, d)):
        raise ValueError(f"{what}: o_out must be fp32 [{B},{T},{H},{d}]")
    tensors = [qp, kp, vp, g, beta, gate, wq, wk, wv] + list(conv_state or []) + \
        ([initial_state] if initial_state is not None else []) + ([o_out] if o_out is not None else [])
    for i, t in enumerate(tensors):
        _contig(f"arg{i}", t)
    dev = _require_gpu(tensors, what)
    L = _lib.lib()
    need = int(L.kda_layer_fwd_workspace(B, T, H, d, K, code))
    if need == 0:
        raise ValueError(f"{what}: unsupported configuration")
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    y = torch.empty((B, T, H * d), dtype=out_dtype, device=dev)
    ht = torch.empty((B, H, d, d), dtype=torch.float32, device=dev) if output_final_state else None
    new = tuple(torch.empty((B, K - 1, H * d), dtype=torch.float32, device=dev) for _ in range(3)) \
        if return_conv_state else (None, None, None)
    bin_ = conv_state if conv_state is not None else (None, None, None)
    rc = L.kda_layer_fwd(_stream(dev), _ptr(qp), _ptr(kp), _ptr(vp), _ptr(g), _ptr(beta), _ptr(gate),
                         _ptr(wq), _ptr(wk), _ptr(wv), *(_ptr(b) for b in bin_), *(_ptr(b) for b in new),
                         _ptr(initial_state), _ptr(ht), _ptr(y), _ptr(o_out), B, T, H, d, K, float(scale), float(eps),
                         code, _OUT_CODES[gate.dtype], _OUT_CODES[out_dtype], _ptr(workspace), need)
    _lib.check(rc, what)
    return y, ht, (new if return_conv_state else None)


def prologue_bwd_workspace_bytes(B, T, H, d, K) -> int:
    """Workspace bytes :func:`kda_prologue_bwd` needs (0 for an unsupported configuration)."""
    return int(_lib.lib().kda_prologue_bwd_workspace(B, T, H, d, K))


def kda_prologue_bwd(qp, kp, vp, wq, wk, wv, dq, dk, dv, conv_state=None, workspace=None):
    """Gradients of :func:`kda_prologue` (the VJP of ``net/kda.py:194-202``
    after the convs of ``:383-389``).

    Inputs as :func:`kda_prologue` plus the cotangents ``dq, dk, dv [B, T, H, d]``.
    Returns fp32 ``((dqp, dkp, dvp) [B, T, H*d], (dwq, dwk, dwv) [K, H*d],
    dconv_state)`` where ``dconv_state`` is three ``[B, K-1, H*d]`` buffer
    gradients (None when ``conv_state`` is None or K == 1).  A row whose
    swish output is all zeros gets a zero L2-norm gradient.
    """
    what = "kda_prologue_bwd"
    if qp.dim() != 3 or kp.shape != qp.shape or vp.shape != qp.shape:
        raise ValueError(f"{what}: qp, kp, vp must share a [B,T,H*d] shape")
    B, T, HD = qp.shape
    if dq.dim() != 4:
        raise ValueError(f"{what}: dq must be [B,T,H,d]")
    H, d = dq.shape[2], dq.shape[3]
    if tuple(dq.shape) != (B, T, H, d) or H * d != HD or dk.shape != dq.shape or dv.shape != dq.shape:
        raise ValueError(f"{what}: dq, dk, dv must be [{B},{T},H,d] with H*d = {HD}")
    if any(t.dtype != torch.float32 for t in (dq, dk, dv)):
        raise ValueError(f"{what}: dq, dk, dv must be fp32")
    if d not in SUPPORTED_HEAD_DIMS:
        raise ValueError(f"{what}: head dim {d} unsupported ({SUPPORTED_HEAD_DIMS})")
    if qp.dtype not in _UT_CODES or kp.dtype != qp.dtype or vp.dtype != qp.dtype:
        raise ValueError(f"{what}: projections must be fp32 or bf16")
    K = wq.shape[0]
    for name, w in (("wq", wq), ("wk", wk), ("wv", wv)):
        if w.dtype != torch.float32 or tuple(w.shape) != (K, HD):
            raise ValueError(f"{what}: {name} must be fp32 [{K},{HD}]")
    if conv_state is not None:
        for st in conv_state:
            if st.dtype != torch.float32 or tuple(st.shape) != (B, K - 1, HD):
                raise ValueError(f"{what}: conv_state buffers must be fp32 [{B},{K - 1},{HD}]")
    tensors = [qp, kp, vp, wq, wk, wv, dq, dk, dv] + list(conv_state or [])
    for i, t in enumerate(tensors):
        _contig(f"arg{i}", t)
    dev = _require_gpu(tensors, what)
    L = _lib.lib()
    need = int(L.kda_prologue_bwd_workspace(B, T, H, d, K))
    if need == 0:
        raise ValueError(f"{what}: unsupported configuration")
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    f32 = torch.float32
    dx = tuple(torch.empty((B, T, HD), dtype=f32, device=dev) for _ in range(3))
    dw = tuple(torch.empty((K, HD), dtype=f32, device=dev) for _ in range(3))
    want_db = conv_state is not None and K > 1
    db = tuple(torch.empty((B, K - 1, HD), dtype=f32, device=dev) for _ in range(3)) if want_db \
        else (None, None, None)
    bin_ = conv_state if conv_state is not None else (None, None, None)
    rc = L.kda_prologue_bwd(_stream(dev), _ptr(qp), _ptr(kp), _ptr(vp), _ptr(wq), _ptr(wk), _ptr(wv),
                            *(_ptr(b) for b in bin_), _ptr(dq), _ptr(dk), _ptr(dv),
                            *(_ptr(t) for t in dx), *(_ptr(t) for t in dw), *(_ptr(t) for t in db),
                            B, T, H, d, K, _UT_CODES[qp.dtype], _ptr(workspace), need)
    _lib.check(rc, what)
    return dx, dw, (db if want_db else None)


def kda_epilogue_bwd(o, gate, dy, eps: float = 1e-6, dgate_dtype=None):
    """Gradients of :func:`kda_epilogue`: ``(do [B, T, H, dv] fp32, dgate [B, T, H*dv])``.

    ``dgate`` is in ``dgate_dtype`` (default: the gate's dtype).
    """
    what = "kda_epilogue_bwd"
    if o.dim() != 4:
        raise ValueError(f"{what}: o must be [B,T,H,dv]")
    B, T, H, dv = o.shape
    if tuple(gate.shape) != (B, T, H * dv) or tuple(dy.shape) != (B, T, H * dv):
        raise ValueError(f"{what}: gate and dy must be [{B},{T},{H * dv}]")
    if dv not in SUPPORTED_HEAD_DIMS:
        raise ValueError(f"{what}: dv={dv} unsupported ({SUPPORTED_HEAD_DIMS})")
    dgate_dtype = gate.dtype if dgate_dtype is None else dgate_dtype
    if any(t not in _UT_CODES for t in (o.dtype, gate.dtype, dy.dtype, dgate_dtype)):
        raise ValueError(f"{what}: dtypes must be fp32 or bf16")
    for name, t in (("o", o), ("gate", gate), ("dy", dy)):
        _contig(name, t)
    dev = _require_gpu([o, gate, dy], what)
    do = torch.empty((B, T, H, dv), dtype=torch.float32, device=dev)
    dgate = torch.empty((B, T, H * dv), dtype=dgate_dtype, device=dev)
    rc = _lib.lib().kda_epilogue_bwd(_stream(dev), _ptr(o), _ptr(gate), _ptr(dy), _ptr(do), _ptr(dgate),
                                     B, T, H, dv, float(eps), _UT_CODES[o.dtype], _UT_CODES[gate.dtype],
                                     _UT_CODES[dy.dtype], _UT_CODES[dgate_dtype])
    _lib.check(rc, what)
    return do, dgate


class _KDALayer(torch.autograd.Function):
    """``(y, final_state)`` of :func:`kda_layer_fwd` with a backward that runs on
    the HIP kernels: the forward keeps the scan's output o (fp32) for the
    epilogue backward; q, k, v are recomputed by the prologue; then epilogue
    backward -> chunked backward -> prologue backward."""

    @staticmethod
    def forward(ctx, qp, kp, vp, g, beta, gate, wq, wk, wv, bq, bk, bv, initial_state, scale, eps):
        conv_state = None if bq is None else (bq, bk, bv)
        B, T, H, d = g.shape
        o = torch.empty((B, T, H, d), dtype=torch.float32, device=qp.device)   # kept for the epilogue backward
        y, ht, _ = kda_layer_fwd(qp, kp, vp, g, beta, gate, wq, wk, wv, conv_state=conv_state,
                                 initial_state=initial_state, scale=scale, eps=eps, return_conv_state=False,
                                 out_dtype=qp.dtype, o_out=o)
        ctx.save_for_backward(qp, kp, vp, g, beta, gate, wq, wk, wv, bq, bk, bv, initial_state, o)
        ctx.scale, ctx.eps = scale, eps
        return y, ht

    @staticmethod
    def backward(ctx, dy, dht):
        qp, kp, vp, g, beta, gate, wq, wk, wv, bq, bk, bv, h0, o = ctx.saved_tensors
        conv_state = None if bq is None else (bq, bk, bv)
        B, T, H, d = g.shape
        if dy is None:
            dy = torch.zeros((B, T, H * d), dtype=torch.float32, device=qp.device)
        dy = dy.contiguous()
        if dy.dtype not in _OUT_CODES:
            dy = dy.float()
        q, k, v, _ = kda_prologue(qp, kp, vp, wq, wk, wv, H, conv_state=conv_state, return_state=False,
                                  out_dtype=qp.dtype)
        do, dgate = kda_epilogue_bwd(o, gate, dy, eps=ctx.eps)
        dht = None if dht is None else dht.float().contiguous()
        dq, dk, dv, dg, dbeta, dh0 = kda_chunk_bwd(q, k, v, g, beta, do, dht=dht, initial_state=h0,
                                                   scale=ctx.scale, need_dh0=ctx.needs_input_grad[12])
        dx, dw, db = kda_prologue_bwd(qp, kp, vp, wq, wk, wv, dq, dk, dv, conv_state=conv_state)
        db = db if db is not None else (None, None, None)
        return (dx[0].to(qp.dtype), dx[1].to(kp.dtype), dx[2].to(vp.dtype), dg.to(g.dtype),
                dbeta.to(beta.dtype), dgate, dw[0], dw[1], dw[2], db[0], db[1], db[2], dh0, None, None)


def kda_layer(qp, kp, vp, g, beta, gate, wq, wk, wv, conv_state=None, initial_state=None,
              scale: float = 1.0, eps: float = 1e-6):
    """Differentiable chunked KDA layer between the projections and ``W_o``:
    ``(y [B, T, H*d] in the projections' dtype, final_state [B, H, d, d] fp32)``.

    The forward is :func:`kda_layer_fwd`; gradients flow to the projections,
    ``g``, ``beta``, the gate logits, the conv taps, the carried conv buffers
    and ``initial_state`` (dense inputs, no ``cu_seqlens``).
    """
    bq, bk, bv = conv_state if conv_state is not None else (None, None, None)
    return _KDALayer.apply(qp, kp, vp, g, beta, gate, wq, wk, wv, bq, bk, bv, initial_state, scale, eps)


def varlen_status(workspace, B, T, H, dk, dv, n_seqs, in_code=_lib.KDA_DTYPE_BF16) -> int:
    """Validation bits of the last varlen call that used ``workspace`` (synchronises)."""
    flags = ctypes.c_int32(0)
    rc = _lib.lib().kda_varlen_status(_stream(workspace.device), _ptr(workspace),
                                      workspace.numel() * workspace.element_size(),
                                      B, T, H, dk, dv, CHUNK, n_seqs, in_code, ctypes.byref(flags))
    _lib.check(rc, "kda_varlen_status")
    return int(flags.value)


def kda_recurrent_step(q, k, v, g, beta, state, scale: float = 1.0, out_dtype=torch.float32):
    """One decode token per chain; ``state [B,H,dk,dv]`` fp32 is updated in place.

    ``q, k, g [B,H,dk]``, ``v [B,H,dv]``, ``beta [B,H]`` (one dtype: bf16, fp16
    or fp32).  Returns ``o [B,H,dv]`` in ``out_dtype``.
    """
    what = "kda_recurrent_step"
    if q.dim() != 3 or k.shape != q.shape or g.shape != q.shape:
        raise ValueError(f"{what}: q, k, g must share a [B,H,dk] shape")
    B, H, dk = q.shape
    if v.dim() != 3 or v.shape[:2] != q.shape[:2]:
        raise ValueError(f"{what}: v must be [B,H,dv]")
    dv = v.shape[2]
    if tuple(beta.shape) != (B, H):
        raise ValueError(f"{what}: beta must be [B,H]")
    _check_dims(dk, dv, what)
    if q.dtype not in _IN_CODES or any(t.dtype != q.dtype for t in (k, v, g, beta)):
        raise ValueError(f"{what}: q, k, v, g, beta must share a dtype in bf16/fp16/fp32")
    if state.dtype != torch.float32 or tuple(state.shape) != (B, H, dk, dv):
        raise ValueError(f"{what}: state must be fp32 [{B},{H},{dk},{dv}]")
    if out_dtype not in _OUT_CODES:
        raise ValueError(f"{what}: out_dtype must be fp32 or bf16")
    for name, t in (("q", q), ("k", k), ("v", v), ("g", g), ("beta", beta), ("state", state)):
        _contig(name, t)
    dev = _require_gpu([q, k, v, g, beta, state], what)
    o = torch.empty((B, H, dv), dtype=out_dtype, device=dev)
    rc = _lib.lib().kda_recurrent_step(_stream(dev), _ptr(q), _ptr(k), _ptr(v), _ptr(g), _ptr(beta),
                                       _ptr(state), _ptr(o), B, H, dk, dv, float(scale),
                                       _IN_CODES[q.dtype], _OUT_CODES[out_dtype])
    _lib.check(rc, what)
    return o


def _cc_check(q, k, v, alpha, beta32, S, tile, chunk, what, dtype_msg):
    """Validates the seam's operands, unbatched (T, H*d) or with a leading batch
    axis (B, T, H*d) -- the vmapped caller of net/model.py:341-347; returns
    (B, T, H, dk, dv, C) with B = 0 for the unbatched form."""
    batched = q.dim() == 3
    if batched:
        if S.dim() != 4:
            raise ValueError(f"{what}: with batched operands S must be (B, H, dk, dv)")
        B, H, dk, dv = S.shape
        T = q.shape[1]
        lead = (B, T)
    else:
        if S.dim() != 3:
            raise ValueError(f"{what}: S must be (H, dk, dv)")
        H, dk, dv = S.shape
        B, T = 0, q.shape[0]
        lead = (T,)
    dt = q.dtype
    if v.dtype != dt or dt != torch.bfloat16:
        raise ValueError(f"{dtype_msg}; got q.dtype={dt}, v.dtype={v.dtype}")
    C = int(chunk)
    if C < 1 or T % C:
        raise ValueError(f"T={T} must be a multiple of the chunk width C={C}")
    if not (1 <= int(tile) <= 16):
        raise ValueError(f"{what}: tile={tile} outside [1, 16]")
    _check_dims(dk, dv, what)
    if (tuple(q.shape) != lead + (H * dk,) or tuple(k.shape) != lead + (H * dk,) or k.dtype != dt
            or tuple(v.shape) != lead + (H * dv,) or tuple(alpha.shape) != lead + (H * dk,)
            or tuple(beta32.shape) != lead + (H * 32,)):
        raise ValueError(f"{what}: shapes must be q,k,alpha ([B,] T,H*dk), v ([B,] T,H*dv), "
                         "beta32 ([B,] T,H*32)")
    if alpha.dtype != torch.float32 or beta32.dtype != torch.float32 or S.dtype != torch.float32:
        raise ValueError(f"{what}: alpha, beta32 and S must be fp32")
    for name, t in (("q", q), ("k", k), ("v", v), ("alpha", alpha), ("beta32", beta32), ("S", S)):
        _contig(name, t)
    return B, T, H, dk, dv, C


def _cc_scan_fwd(q, k, v, alpha, beta32, S, tile, chunk):
    B, T, H, dk, dv, C = _cc_check(q, k, v, alpha, beta32, S, tile, chunk, "cc_scan",
                                   "persistent kernel consumes bf16 q/k/v")
    dev = _require_gpu([q, k, v, alpha, beta32, S], "cc_scan")
    L = _lib.lib()
    nb = max(B, 1)
    ws_bytes = int(L.kda_cc_scan_batched_workspace(nb, T, H, dk, dv, C))
    workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    o = torch.empty(q.shape[:-1] + (H * dv,), dtype=torch.float32, device=dev)
    S_new = torch.empty_like(S)
    rc = L.kda_cc_scan_batched(_stream(dev), _ptr(q), _ptr(k), _ptr(v), _ptr(alpha), _ptr(beta32), _ptr(S),
                               _ptr(o), _ptr(S_new), nb, T, H, dk, dv, int(tile), C, _ptr(workspace), ws_bytes)
    _lib.check(rc, "cc_scan")
    return o, S_new


def cc_scan_bwd(q, k, v, alpha, beta32, S, do, dS=None, tile: int = 16, chunk: int = 32):
    """The seam's backward rule ``kernel_bwd`` (``net/kernels/kda_cc_fused_persist.py:1710``).

    ``(q, k, v, alpha, beta32, S)`` as :func:`cc_scan`, ``do ([B,] T, H*dv)`` and
    ``dS ([B,] H, dk, dv)`` (None = 0) the cotangents of ``o`` and ``S_new``.
    Returns ``(dq, dk, dv, dalpha, dbeta32, dS_in)`` in the primal dtypes:
    bf16 ``dq, dk, dv``, fp32 ``dalpha`` (``= d(log alpha) / alpha``),
    ``dbeta32`` (the beta cotangent / 32 on each of the 32 columns) and
    ``dS_in``.
    """
    what = "cc_scan_bwd"
    B, T, H, dk, dv, C = _cc_check(q, k, v, alpha, beta32, S, tile, chunk, what,
                                   "persistent backward kernel consumes bf16 q/k/v (the same operand "
                                   "path as the forward kernel)")
    if tuple(do.shape) != tuple(q.shape[:-1]) + (H * dv,):
        raise ValueError(f"{what}: do must be ([B,] T, H*dv) = {tuple(q.shape[:-1]) + (H * dv,)}")
    do = do.float().contiguous()
    if dS is None:
        dS = torch.zeros_like(S)
    if tuple(dS.shape) != tuple(S.shape):
        raise ValueError(f"{what}: dS must be shaped as S ([B,] H, dk, dv)")
    dS = dS.float().contiguous()
    dev = _require_gpu([q, k, v, alpha, beta32, S, do, dS], what)
    L = _lib.lib()
    nb = max(B, 1)
    ws_bytes = int(L.kda_cc_scan_bwd_batched_workspace(nb, T, H, dk, dv, C))
    workspace = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    dq = torch.empty_like(q)
    dk_ = torch.empty_like(k)
    dv_ = torch.empty_like(v)
    dalpha = torch.empty_like(alpha)
    dbeta32 = torch.empty_like(beta32)
    dS_in = torch.empty_like(S)
    rc = L.kda_cc_scan_bwd_batched(_stream(dev), _ptr(q), _ptr(k), _ptr(v), _ptr(alpha), _ptr(beta32), _ptr(S),
                                   _ptr(do), _ptr(dS), _ptr(dq), _ptr(dk_), _ptr(dv_), _ptr(dalpha),
                                   _ptr(dbeta32), _ptr(dS_in), nb, T, H, dk, dv, int(tile), C,
                                   _ptr(workspace), ws_bytes)
    _lib.check(rc, what)
    return dq, dk_, dv_, dalpha, dbeta32, dS_in


class _CCScan(torch.autograd.Function):
    """``cc_scan`` with :func:`cc_scan_bwd` as its VJP, as the reference's
    ``custom_vjp`` (``net/kernels/kda_cc_fused_persist.py:895-911``)."""

    @staticmethod
    def forward(ctx, q, k, v, alpha, beta32, S, tile, chunk):
        o, S_new = _cc_scan_fwd(q, k, v, alpha, beta32, S, tile, chunk)
        ctx.save_for_backward(q, k, v, alpha, beta32, S)
        ctx.tile, ctx.chunk = tile, chunk
        return o, S_new

    @staticmethod
    def backward(ctx, do, dS):
        q, k, v, alpha, beta32, S = ctx.saved_tensors
        if do is None:
            do = torch.zeros(v.shape, dtype=torch.float32, device=q.device)
        grads = cc_scan_bwd(q, k, v, alpha, beta32, S, do, dS, tile=ctx.tile, chunk=ctx.chunk)
        return (*grads, None, None)


def cc_scan(q, k, v, alpha, beta32, S, tile: int = 16, chunk: int = 32):
    """The reference seam ``cc_scan`` (``net/kernels/kda_cc_fused_persist.py:920``).

    ``q, k (T, H*dk)`` bf16, ``v (T, H*dv)`` bf16, ``alpha (T, H*dk)`` fp32,
    ``beta32 (T, H*32)`` fp32, ``S (H, dk, dv)`` fp32.  Returns
    ``(o (T, H*dv) fp32, S_new (H, dk, dv) fp32)``.  Every operand may carry a
    leading batch axis B (the vmapped caller, ``net/model.py:341-347``): the
    batch then runs in one launch.  Raises ``ValueError`` for
    a non-bf16 q/v (``:737-740``), ``T % chunk != 0`` (``:741-742``) or an
    unsupported configuration (``:743-749``), ``RuntimeError`` without a GPU.
    Differentiable: gradients reach all six inputs through
    :func:`cc_scan_bwd`, like the reference's ``custom_vjp``.
    """
    return _CCScan.apply(q, k, v, alpha, beta32, S, tile, chunk)
