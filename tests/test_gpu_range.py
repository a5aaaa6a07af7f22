"""fp16 operand range of the 16-bit forward (kda_chunk_fwd's precondition).

16-bit inputs run on fp16 matrix-core operands.  Inside the supported range
(unit-norm q, k; |v|, the state and U below 2^15) the result meets the bf16
bar at any scale; outside it the state kernels see non-finite values and the
call's status word says so (kda_chunk_fwd_status), so a caller gets a typed
error (check_finite) and never a silent inf.  fp32 inputs (exact mode) have
fp32 range.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle import inputs, kda_oracle as K
from tests.kda_testutil import TOL, assert_close, to_dev

pytestmark = pytest.mark.gpu


def _case(v_scale=1.0, h0_std=0.0, B=1, T=300, H=2, d=128, seed=41):
    x = inputs.make_inputs(B, T, H, d, d, seed=seed, dtype="bf16", h0_std=h0_std)
    x["v"] = torch.from_numpy(x["v"]).mul(v_scale).to(torch.bfloat16).float().numpy()
    return x


def _run(cuda, x, dt=torch.bfloat16, check=False):
    import axiom_amd
    t = {n: to_dev(x[n], dt, cuda) for n in ("q", "k", "v", "g", "beta")}
    h0 = to_dev(x["h0"], torch.float32, cuda) if "h0" in x else None
    o, ht = axiom_amd.kda_chunk_fwd(t["q"], t["k"], t["v"], t["g"], t["beta"], initial_state=h0,
                                    check_finite=check)
    torch.cuda.synchronize()
    return o, ht


def test_large_in_range_values_are_exact_to_the_bar(cuda):
    """|v| scaled by 300 (values up to ~1.5e3) and h0 ~ N(0, 30^2): inside the
    fp16 range; relative errors are those of unit-scale inputs."""
    s = 300.0
    x = _case(v_scale=s, h0_std=30.0)
    o, ht = _run(cuda, x, check=True)
    o_ref, ht_ref = K.chunk_fwd(x["q"], x["k"], x["v"], x["g"], x["beta"], h0=x["h0"], chunk=64)
    assert_close("o", o, o_ref, (TOL["bf16"][0], TOL["bf16"][1] * s))
    assert_close("ht", ht, ht_ref, (TOL["bf16"][0], TOL["bf16"][1] * s))


@pytest.mark.parametrize("what", ["v", "h0"])
def test_out_of_range_is_a_typed_error(cuda, what):
    """|v| ~ 1e5 or |h0| ~ 1e5: beyond fp16; check_finite raises ValueError, and
    without it the status query reports the non-finite result."""
    import axiom_amd
    from axiom_amd import _lib, kda as kmod
    x = _case(v_scale=1e5) if what == "v" else _case(h0_std=1e5)
    with pytest.raises(ValueError, match="non-finite"):
        _run(cuda, x, check=True)
    # the same call without the check, through an explicit workspace
    B, T, H, d = x["q"].shape
    ws = torch.empty(kmod.chunk_fwd_workspace_bytes(B, T, H, d, d), dtype=torch.uint8, device=cuda)
    t = {n: to_dev(x[n], torch.bfloat16, cuda) for n in ("q", "k", "v", "g", "beta")}
    h0 = to_dev(x["h0"], torch.float32, cuda) if "h0" in x else None
    o, ht = axiom_amd.kda_chunk_fwd(t["q"], t["k"], t["v"], t["g"], t["beta"], initial_state=h0, workspace=ws)
    assert not (torch.isfinite(o).all() and torch.isfinite(ht).all())
    flags = ctypes.c_int32(0)
    rc = _lib.lib().kda_chunk_fwd_status(ctypes.c_void_p(torch.cuda.current_stream(cuda).cuda_stream),
                                         ctypes.c_void_p(ws.data_ptr()), ws.numel(), B, T, H, d, d, 64, 0,
                                         _lib.KDA_DTYPE_BF16, ctypes.byref(flags))
    assert rc == 0 and flags.value & _lib.KDA_STATUS_NONFINITE
    # a good call on the same workspace clears the word
    good = _case()
    tg = {n: to_dev(good[n], torch.bfloat16, cuda) for n in ("q", "k", "v", "g", "beta")}
    axiom_amd.kda_chunk_fwd(tg["q"], tg["k"], tg["v"], tg["g"], tg["beta"], workspace=ws)
    rc = _lib.lib().kda_chunk_fwd_status(ctypes.c_void_p(torch.cuda.current_stream(cuda).cuda_stream),
                                         ctypes.c_void_p(ws.data_ptr()), ws.numel(), B, T, H, d, d, 64, 0,
                                         _lib.KDA_DTYPE_BF16, ctypes.byref(flags))
    assert rc == 0 and flags.value == 0


def test_fp32_inputs_have_fp32_range(cuda):
    """The same out-of-fp16-range values as fp32 inputs (exact mode): finite
    and at the fp32 bar (relative to the scale)."""
    x = _case(v_scale=1e5)
    x = {n: np.asarray(a, np.float32) for n, a in x.items()}
    o, ht = _run(cuda, x, dt=torch.float32, check=True)
    o_ref, ht_ref = K.chunk_fwd(x["q"], x["k"], x["v"], x["g"], x["beta"], chunk=64)
    assert_close("o", o, o_ref, (TOL["fp32"][0], TOL["fp32"][1] * 1e5))
    assert_close("ht", ht, ht_ref, (TOL["fp32"][0], TOL["fp32"][1] * 1e5))
