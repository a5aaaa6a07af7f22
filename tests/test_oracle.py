"""Pins of the CPU oracle (no GPU).

The reference ships no golden vectors for this path and its JAX code cannot
run here, so the oracle is pinned by what the mathematics fixes and by the
reference's own cross-form tests:

* closed forms of the delta rule (``net/kda.py:298-310``) and a literal,
  scalar implementation of Eq. 1 (``net/kda-formulas.md:12-21``);
* chunked WY/UT == recurrence for C in {16, 32, 64, 128} within the
  reference's 1e-4 bar (``net/tests/test_kda_chunked_cc.py:189-208``), chunk
  invariance, chunk-boundary states (``:413-427``), T < C and ragged tails
  (``:270-288``);
* tile-wise scores == brute-force ``(C, C, dk)`` decay tensor at the
  strongest decay (``:221-247``);
* UT solve == ``scipy.linalg.solve_triangular`` and the Neumann product
  (``net/kernels/kda_ut_solve.py:20-27``, envelope
  ``net/tests/test_kernel_kda_ut_solve.py:105-127``);
* varlen == per-sequence runs; decode steps == chunked forward;
* mutation tests: each plausible mistake planted into a copy of the oracle
  (dropped term, sign flip, transposed operand, off-by-one decay, wrong mask)
  makes at least one of these pins fail.
"""

from __future__ import annotations

import numpy as np
import pytest
import scipy.linalg
import torch

from oracle import inputs, kda_oracle as K


def _small(B=2, T=96, H=3, dk=16, dv=12, seed=0, h0=0.1, dtype="fp32"):
    return inputs.make_inputs(B, T, H, dk, dv, seed=seed, dtype=dtype, h0_std=h0)


# ---------------------------------------------------------------------------
# closed forms and a literal Eq. 1
# ---------------------------------------------------------------------------


def _eq1_scalar(q, k, v, g, beta, S):
    """Eq. 1 literally with Python scalars: S <- (I - b k k^T) Diag(a) S + b k v^T; o = S^T q."""
    dk, dv = len(k), len(v)
    a = [np.exp(float(x)) for x in g]
    DS = [[a[i] * S[i][j] for j in range(dv)] for i in range(dk)]
    M = [[(1.0 if i == m else 0.0) - beta * k[i] * k[m] for m in range(dk)] for i in range(dk)]
    out = [[sum(M[i][m] * DS[m][j] for m in range(dk)) + beta * k[i] * v[j] for j in range(dv)]
           for i in range(dk)]
    o = [sum(out[i][j] * q[i] for i in range(dk)) for j in range(dv)]
    return np.array(o), np.array(out)


def test_decode_step_equals_literal_eq1():
    d = inputs.make_inputs(1, 5, 1, 4, 3, seed=3, dtype="fp32", h0_std=0.5)
    S = d["h0"][0, 0].astype(np.float64)
    S_lit = S.tolist()
    for t in range(5):
        q, k, v, g, b = (d[n][0, t, 0] for n in ("q", "k", "v", "g", "beta"))
        o, S = K.decode_step(q, k, v, g, b, S)
        o_l, S_l = _eq1_scalar(q.tolist(), k.tolist(), v.tolist(), g.tolist(), float(b), S_lit)
        S_lit = S_l.tolist()
        np.testing.assert_allclose(o, o_l, rtol=0, atol=1e-13)
        np.testing.assert_allclose(S, S_l, rtol=0, atol=1e-13)


def test_closed_form_beta_zero_is_pure_decay():
    d = _small(B=1, T=1, H=2)
    S = d["h0"].astype(np.float64)
    q, k, v, g = (d[n][:, 0] for n in ("q", "k", "v", "g"))
    o, S1 = K.decode_step(q, k, v, g, np.zeros((1, 2)), S)
    np.testing.assert_allclose(S1, np.exp(g.astype(np.float64))[..., None] * S, atol=1e-15)
    np.testing.assert_allclose(o, np.einsum("bhd,bhde->bhe", q, S1), atol=1e-14)


def test_closed_form_identity():
    d = _small(B=1, T=1, H=2)
    S = d["h0"].astype(np.float64)
    q, k, v = (d[n][:, 0] for n in ("q", "k", "v"))
    _, S1 = K.decode_step(q, k, v, np.zeros_like(q), np.zeros((1, 2)), S)
    np.testing.assert_array_equal(S1, S)


def test_closed_form_full_forget_overwrites():
    d = _small(B=1, T=1, H=2)
    S = d["h0"].astype(np.float64)
    q, k, v, b = (d[n][:, 0] for n in ("q", "k", "v", "beta"))
    _, S1 = K.decode_step(q, k, v, np.full_like(q, -1e4), b, S)
    np.testing.assert_allclose(S1, b[..., None, None] * k[..., :, None] * v[..., None, :], atol=1e-15)


def test_closed_form_single_token_from_zero():
    d = _small(B=2, T=1, H=3)
    o, ht = K.recurrent_fwd(d["q"], d["k"], d["v"], d["g"], d["beta"])
    kq = np.sum(d["k"][:, 0].astype(np.float64) * d["q"][:, 0], -1)
    np.testing.assert_allclose(o[:, 0], (d["beta"][:, 0] * kq)[..., None] * d["v"][:, 0], atol=1e-14)
    oc, _ = K.chunk_fwd(d["q"], d["k"], d["v"], d["g"], d["beta"], chunk=64)
    np.testing.assert_allclose(oc.numpy()[:, 0], o[:, 0], atol=1e-14)


def test_closed_form_orthonormal_keys_store_exactly():
    rng = np.random.default_rng(0)
    dk, dv, T = 16, 5, 10
    Q, _ = np.linalg.qr(rng.standard_normal((dk, dk)))
    k = Q[:, :T].T[None, :, None, :]                      # T orthonormal keys
    v = rng.standard_normal((1, T, 1, dv))
    q = rng.standard_normal((1, T, 1, dk))
    g = np.zeros((1, T, 1, dk))
    beta = np.ones((1, T, 1))
    for S in (K.recurrent_fwd(q, k, v, g, beta)[1],
              K.chunk_fwd(q, k, v, g, beta, chunk=4)[1].numpy()):
        recalled = np.einsum("td,de->te", k[0, :, 0], S[0, 0])
        np.testing.assert_allclose(recalled, v[0, :, 0], atol=1e-12)


# ---------------------------------------------------------------------------
# chunked form against the recurrence (the reference's own parity ladder)
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("C", [16, 32, 64, 128])
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_chunked_equals_recurrent(C, seed):
    d = _small(T=150, seed=seed)
    o_r, s_r = K.recurrent_fwd(d["q"], d["k"], d["v"], d["g"], d["beta"], h0=d["h0"])
    o_c, s_c = K.chunk_fwd(d["q"], d["k"], d["v"], d["g"], d["beta"], h0=d["h0"], chunk=C)
    assert K.max_abs(o_c.numpy(), o_r) <= 1e-10
    assert K.max_abs(s_c.numpy(), s_r) <= 1e-10
    o32, s32 = K.chunk_fwd(d["q"], d["k"], d["v"], d["g"], d["beta"], h0=d["h0"], chunk=C,
                           dtype=torch.float32)
    assert K.max_abs(o32.numpy(), o_r) <= 1e-4          # the reference's fp32 bar
    assert K.max_abs(s32.numpy(), s_r) <= 1e-4


def test_chunk_boundary_states_equal_recurrence():
    d = _small(B=1, T=128, seed=4)
    _, _, states = K.chunk_fwd(d["q"], d["k"], d["v"], d["g"], d["beta"], h0=d["h0"], chunk=32,
                               return_chunk_states=True)
    for n in range(4):
        t = 32 * n
        _, s_t = K.recurrent_fwd(d["q"][:, :t], d["k"][:, :t], d["v"][:, :t], d["g"][:, :t],
                                 d["beta"][:, :t], h0=d["h0"])
        assert K.max_abs(states[:, :, n].numpy(), s_t) <= 1e-10


@pytest.mark.parametrize("T", [1, 5, 63, 64, 65, 100])
def test_short_and_ragged_T(T):
    d = _small(B=1, T=T, seed=T)
    o_r, s_r = K.recurrent_fwd(d["q"], d["k"], d["v"], d["g"], d["beta"], h0=d["h0"])
    o_c, s_c = K.chunk_fwd(d["q"], d["k"], d["v"], d["g"], d["beta"], h0=d["h0"], chunk=64)
    assert K.max_abs(o_c.numpy(), o_r) <= 1e-10
    assert K.max_abs(s_c.numpy(), s_r) <= 1e-10


def test_strong_decay_stays_finite_and_exact():
    """|g| at the reference's g_min = -5 bound: the tile anchoring must not overflow."""
    d = _small(B=1, T=128, seed=9)
    d["g"] = np.full_like(d["g"], -4.99)
    o_r, s_r = K.recurrent_fwd(d["q"], d["k"], d["v"], d["g"], d["beta"], h0=d["h0"])
    o_c, s_c = K.chunk_fwd(d["q"], d["k"], d["v"], d["g"], d["beta"], h0=d["h0"], chunk=128)
    assert np.all(np.isfinite(o_c.numpy()))
    assert K.max_abs(o_c.numpy(), o_r) <= 1e-10


# ---------------------------------------------------------------------------
# scores and UT solve
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("strict", [False, True])
def test_tilewise_scores_equal_bruteforce(strict):
    rng = np.random.default_rng(1)
    N, C, dk = 3, 64, 16
    row = torch.tensor(rng.standard_normal((N, C, dk)))
    col = torch.tensor(rng.standard_normal((N, C, dk)))
    g = torch.full((N, C, dk), -5.0) * torch.tensor(rng.uniform(0.5, 1.0, (N, C, dk)))
    G = torch.cumsum(g, 1)
    got = K.cc_scores(row, col, G, 16, strict)
    E = torch.exp(torch.clamp(G[:, :, None, :] - G[:, None, :, :], max=0.0))
    ref = torch.einsum("ncid,ncd,nid->nci", E, row, col)
    mask = torch.tril(torch.ones(C, C), diagonal=-1 if strict else 0).bool()
    ref = torch.where(mask, ref, torch.zeros(()))
    assert float((got - ref).abs().max() / ref.abs().max()) <= 1e-12


def test_ut_solve_equals_scipy_and_neumann():
    rng = np.random.default_rng(2)
    C = 64
    L = np.tril(rng.uniform(-1.0, 1.0, (2, C, C)), -1)      # the KDA envelope |L| <= 1
    Tm = K.ut_solve(torch.tensor(L)).numpy()
    B = rng.standard_normal((C, 7))
    for n in range(2):
        x = scipy.linalg.solve_triangular(np.eye(C) + L[n], B, lower=True, unit_diagonal=True)
        np.testing.assert_allclose(Tm[n] @ B, x, rtol=1e-9, atol=1e-9)
        prod = np.eye(C) - L[n]                            # (I - L)(I + L^2)(I + L^4)...
        P = L[n] @ L[n]
        for _ in range(5):
            prod = prod @ (np.eye(C) + P)
            P = P @ P
        np.testing.assert_allclose(prod, Tm[n], rtol=1e-9, atol=1e-9)


# ---------------------------------------------------------------------------
# varlen and decode invariants
# ---------------------------------------------------------------------------


def test_varlen_packed_equals_per_sequence():
    lengths = [3, 64, 0, 90, 17]
    cu = inputs.cu_seqlens_from_lengths(lengths)
    d = inputs.make_inputs(1, int(cu[-1]), 2, 16, 8, seed=5, dtype="fp32", h0_std=0.1,
                           n_states=len(lengths))
    o_c, h_c = K.chunk_fwd(d["q"], d["k"], d["v"], d["g"], d["beta"], h0=d["h0"], cu_seqlens=cu)
    o_r, h_r = K.recurrent_fwd(d["q"], d["k"], d["v"], d["g"], d["beta"], h0=d["h0"], cu_seqlens=cu)
    assert K.max_abs(o_c.numpy(), o_r) <= 1e-10
    assert K.max_abs(h_c.numpy(), h_r) <= 1e-10
    np.testing.assert_array_equal(h_c[2].numpy(), d["h0"][2])   # empty sequence keeps h0
    for i in range(len(lengths)):
        a, b = int(cu[i]), int(cu[i + 1])
        if a == b:
            continue
        oi, hi = K.chunk_fwd(*(d[n][:, a:b] for n in ("q", "k", "v", "g", "beta")), h0=d["h0"][i:i + 1])
        assert K.max_abs(o_c.numpy()[:, a:b], oi.numpy()) <= 1e-12
        assert K.max_abs(h_c.numpy()[i], hi.numpy()[0]) <= 1e-12


def test_decode_steps_equal_chunked():
    d = _small(B=2, T=40, seed=6)
    o_c, s_c = K.chunk_fwd(d["q"], d["k"], d["v"], d["g"], d["beta"], h0=d["h0"], chunk=16)
    steps = {n: np.moveaxis(d[n], 1, 0) for n in ("q", "k", "v", "g", "beta")}
    o_d, s_d = K.decode_steps(steps["q"], steps["k"], steps["v"], steps["g"], steps["beta"], d["h0"])
    assert K.max_abs(o_c.numpy(), np.moveaxis(o_d, 0, 1)) <= 1e-10
    assert K.max_abs(s_c.numpy(), s_d) <= 1e-10


@pytest.mark.parametrize("scale", [1.0, 0.7])
def test_batched_decode_steps_equal_the_chunked_forward(scale):
    """decode_steps_torch (the batched form the full-size decode check uses)
    against the chunked oracle over the same tokens, and against the numpy
    steps; a step that skips the decay of the read fails the first check."""
    d = _small(B=2, T=40, seed=16)
    # (the chunked oracle applies the scale in fp32: ~1e-8 apart from fp64 at 0.7)
    o_c, s_c = K.chunk_fwd(d["q"], d["k"], d["v"], d["g"], d["beta"], h0=d["h0"], chunk=16, scale=scale)
    steps = {n: np.moveaxis(d[n], 1, 0) for n in ("q", "k", "v", "g", "beta")}
    o_t, s_t = K.decode_steps_torch(steps["q"], steps["k"], steps["v"], steps["g"], steps["beta"], d["h0"], scale)
    bar = 1e-10 if scale == 1.0 else 1e-7
    assert K.max_abs(o_c.numpy(), np.moveaxis(o_t, 0, 1)) <= bar
    assert K.max_abs(s_c.numpy(), s_t) <= 1e-10
    o_n, s_n = K.decode_steps(steps["q"], steps["k"], steps["v"], steps["g"], steps["beta"], d["h0"], scale)
    assert K.max_abs(o_n, o_t) <= 1e-12 and K.max_abs(s_n, s_t) <= 1e-12
    # planted: the decay dropped (g taken as zero)
    o_m, _ = K.decode_steps_torch(steps["q"], steps["k"], steps["v"], np.zeros_like(steps["g"]), steps["beta"],
                                  d["h0"], scale)
    assert K.max_abs(o_c.numpy(), np.moveaxis(o_m, 0, 1)) > 1e-3


# ---------------------------------------------------------------------------
# mutation tests: a planted mistake must fail a pin
# ---------------------------------------------------------------------------


def _chunk_pin_fails(monkeypatch, mutated_step) -> bool:
    monkeypatch.setattr(K, "chunk_step", mutated_step)
    d = _small(T=150, seed=1)
    o_r, s_r = K.recurrent_fwd(d["q"], d["k"], d["v"], d["g"], d["beta"], h0=d["h0"])
    o_c, s_c = K.chunk_fwd(d["q"], d["k"], d["v"], d["g"], d["beta"], h0=d["h0"], chunk=32)
    return K.max_abs(o_c.numpy(), o_r) > 1e-4 or K.max_abs(s_c.numpy(), s_r) > 1e-4


def _make_step(variant):
    def step(q, k, v, G, beta, S, tile=16):
        if variant == "exclusive_cumsum":
            G = G - (G[:, :1, :] * 0 + torch.diff(G, dim=1, prepend=torch.zeros_like(G[:, :1])))
        aqk = K.cc_scores(q, k, G, tile, strict=False)
        akk = K.cc_scores(k, k, G, tile, strict=(variant != "nonstrict_akk"))
        L = akk * beta[:, :, None]
        gamma = torch.exp(G)
        xw = gamma * k * beta[:, :, None]
        vw = v * beta[:, :, None]
        Tm = K.ut_solve(L)
        w = Tm @ xw
        u = Tm @ vw
        v_tilde = (u + w @ S) if variant == "sign_flip" else (u - w @ S)
        A = aqk.transpose(1, 2) if variant == "transposed_aqk" else aqk
        o = (gamma * q) @ S + (0 if variant == "drop_intra" else A @ v_tilde)
        lam = torch.exp(torch.clamp(G[:, -1:, :] - G, max=0.0))
        S_new = gamma[:, -1, :, None] * S + (lam * k).transpose(1, 2) @ v_tilde
        return o, S_new
    return step


@pytest.mark.parametrize("variant", ["drop_intra", "sign_flip", "transposed_aqk",
                                     "exclusive_cumsum", "nonstrict_akk"])
def test_mutated_chunk_oracle_is_caught(monkeypatch, variant):
    assert not _chunk_pin_fails(monkeypatch, _make_step("none")), "unmutated step must pass"
    assert _chunk_pin_fails(monkeypatch, _make_step(variant)), f"mutation {variant} not caught"


def test_mutated_decode_is_caught(monkeypatch):
    """Reading against the undecayed S (a plausible slip) must fail the literal-Eq.1 pin."""
    def bad(q, k, v, g, beta, S, scale=1.0):
        q = np.asarray(q, np.float64) * scale
        k, v, S = (np.asarray(x, np.float64) for x in (k, v, S))
        alpha = np.exp(np.asarray(g, np.float64))
        beta = np.asarray(beta, np.float64)
        read = np.einsum("...d,...de->...e", k, S)        # missing alpha
        S_new = alpha[..., :, None] * S + beta[..., None, None] * k[..., :, None] * (v - read)[..., None, :]
        return np.einsum("...d,...de->...e", q, S_new), S_new
    monkeypatch.setattr(K, "decode_step", bad)
    with pytest.raises(AssertionError):
        test_decode_step_equals_literal_eq1()


# ---------------------------------------------------------------------------
# per-chunk intermediates (the GPU workspace is checked against these)
# ---------------------------------------------------------------------------


def _rebuild_from_intermediates(it, h0):
    """o and the final state from the per-chunk W, U, Aqk, gamma*q, lambda*k,
    gamma_C alone: v~ = U - W S, o = (gamma q) S + Aqk v~,
    S' = gamma_C S + (lambda k)^T v~ (the state recurrence of net/kda.py:689-702)."""
    B, H, n, C, dv = it["U"].shape
    S = np.array(h0, np.float64)
    o = np.zeros((B, H, n, C, dv))
    for i in range(n):
        vt = it["U"][:, :, i] - it["W"][:, :, i] @ S
        o[:, :, i] = it["GQ"][:, :, i] @ S + it["Aqk"][:, :, i] @ vt
        S = it["GC"][:, :, i][..., None] * S + np.swapaxes(it["LK"][:, :, i], -1, -2) @ vt
    return o, S


def _intermediates_case(T=150, C=32, dk=16, dv=12, seed=4):
    d = _small(T=T, dk=dk, dv=dv, seed=seed)
    it = K.chunk_intermediates(d["q"], d["k"], d["v"], d["g"], d["beta"], chunk=C)
    o_r, s_r = K.recurrent_fwd(d["q"], d["k"], d["v"], d["g"], d["beta"], h0=d["h0"])
    return d, it, o_r, s_r


def _rebuild_error(d, it, o_r, s_r):
    o, S = _rebuild_from_intermediates(it, d["h0"])
    B, H, n, C, dv = o.shape
    T = o_r.shape[1]
    o = np.transpose(o.reshape(B, H, n * C, dv), (0, 2, 1, 3))[:, :T]
    return max(K.max_abs(o, o_r), K.max_abs(S, s_r))


@pytest.mark.parametrize("C", [16, 32, 64])
def test_chunk_intermediates_rebuild_the_recurrence(C):
    """The per-chunk intermediates alone reproduce the token recurrence (fp64),
    ragged tail included (T = 150 is not a multiple of C)."""
    d, it, o_r, s_r = _intermediates_case(C=C)
    assert _rebuild_error(d, it, o_r, s_r) <= 1e-10


def test_chunk_intermediates_T_inverts_I_plus_L():
    """T (I + L) = I with L built by brute force from its definition
    L[c,i] = beta_c sum_d k_c k_i exp(G_c - G_i), c > i (net/kda.py:678-681)."""
    d = _small(T=64, dk=16, dv=12, seed=5)
    it = K.chunk_intermediates(d["q"], d["k"], d["v"], d["g"], d["beta"], chunk=32)
    B, T, H, dk = d["k"].shape
    for b in range(B):
        for h in range(H):
            for n in range(2):
                sl = slice(32 * n, 32 * n + 32)
                k = d["k"][b, sl, h].astype(np.float64)
                G = np.cumsum(d["g"][b, sl, h].astype(np.float64), axis=0)
                beta = d["beta"][b, sl, h].astype(np.float64)
                L = np.zeros((32, 32))
                for c in range(32):
                    for i in range(c):
                        L[c, i] = beta[c] * np.sum(k[c] * k[i] * np.exp(G[c] - G[i]))
                Tm = it["T"][b, h, n]
                np.testing.assert_allclose(Tm @ (np.eye(32) + L), np.eye(32), rtol=0, atol=1e-12)


@pytest.mark.parametrize("mistake", ["lk_transposed", "gq_exclusive", "aqk_strict", "w_without_beta",
                                     "gc_first_row", "u_shifted_chunk"])
def test_mutated_intermediates_are_caught(mistake):
    """A plausible slip in chunk_intermediates fails the rebuild pin.  The
    transposed lambda*k needs a square [C, dk] block, so that case runs at
    C = dk = 16."""
    C = 16 if mistake == "lk_transposed" else 32
    d, it, o_r, s_r = _intermediates_case(C=C)
    assert _rebuild_error(d, it, o_r, s_r) <= 1e-10
    it = {n: v.copy() for n, v in it.items()}
    if mistake == "lk_transposed":
        it["LK"] = np.swapaxes(it["LK"], -1, -2).copy()
    elif mistake == "gq_exclusive":
        # gamma of the previous row (exclusive cumsum) instead of the row's own
        g = np.transpose(np.asarray(d["g"], np.float64), (0, 2, 1, 3))
        B, H, n, Cc, dk = it["GQ"].shape
        gp = np.zeros((B, H, n * Cc, dk))
        gp[:, :, :g.shape[2]] = g
        it["GQ"] = it["GQ"] * np.exp(-gp.reshape(B, H, n, Cc, dk))
    elif mistake == "aqk_strict":
        it["Aqk"] = np.tril(it["Aqk"], -1)
    elif mistake == "w_without_beta":
        beta = np.transpose(np.asarray(d["beta"], np.float64), (0, 2, 1))
        B, H, n, Cc, dk = it["W"].shape
        bp = np.ones((B, H, n * Cc))
        bp[:, :, :beta.shape[2]] = beta
        # undo the beta scaling of the right-hand side (beta > 0 on every real row)
        it["W"] = it["T"] @ (np.linalg.solve(it["T"], it["W"]) / bp.reshape(B, H, n, Cc)[..., None])
    elif mistake == "gc_first_row":
        it["GC"] = it["GQ"][..., 0, :] * 0 + np.exp(np.transpose(np.asarray(d["g"], np.float64), (0, 2, 1, 3))
                                                    [:, :, ::C][:, :, :it["GC"].shape[2]])
    elif mistake == "u_shifted_chunk":
        it["U"] = np.roll(it["U"], 1, axis=2)
    assert _rebuild_error(d, it, o_r, s_r) > 1e-4, f"mistake {mistake} not caught"


# ---------------------------------------------------------------------------
# tile width rule
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("g_min,expect", [(-5.0, 16), (-10.0, 8), (0.0, 16), (-3.0, 16), (-20.0, 4),
                                          (-30.0, 2), (-100.0, 1)])
def test_cc_tile_values(g_min, expect):
    """net/kda.py:577-585: the widest tile (at most 16) whose column factor
    exp(|g_min| * tile) stays inside the exponent budget of 80, at least 1."""
    t = K.cc_tile(g_min)
    assert t == expect
    step = abs(g_min)
    assert 1 <= t <= 16
    if t > 1:
        assert t * step <= 80.0
    assert t == 16 or (t + 1) * step > 80.0 or t == 1
