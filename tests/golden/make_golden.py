"""Write the golden fixtures of the KDA hot path (``tests/golden/*.npz``).

The reference holds no golden vectors for this path (its tests draw inputs
from ``jax.random`` at run time), so these fixtures freeze inputs drawn by
``oracle.inputs`` and the outputs of the float64 token-by-token recurrence
(``oracle.kda_oracle.recurrent_fwd`` / ``decode_steps``: the delta rule of
``net/kda.py:298-310`` with the read-out of ``net/kda.py:293``).  The
recurrence shares no code with the chunked algorithm, so a fixture checks the
chunked oracle and the HIP kernels against an independent statement of the
math.

Storage: bf16 inputs as their uint16 bit patterns, fp32 inputs and every
expected output as float32, int32 offsets as int32.

Run from the repository root:  python -m tests.golden.make_golden
"""

from __future__ import annotations

from pathlib import Path

import numpy as np

from oracle import inputs, kda_oracle as K

HERE = Path(__file__).resolve().parent


def _pack(d, prec):
    out = {}
    for name in ("q", "k", "v", "g", "beta"):
        x = np.ascontiguousarray(d[name], np.float32)
        out[name] = inputs.bf16_bits(x) if prec == "bf16" else x
    if "h0" in d:
        out["h0"] = np.ascontiguousarray(d["h0"], np.float32)
    return out


def dense_case(name, B, T, H, dk, seed, prec, h0_std=0.0):
    d = inputs.make_inputs(B, T, H, dk, dk, seed=seed, dtype=prec, h0_std=h0_std)
    o, ht = K.recurrent_fwd(d["q"], d["k"], d["v"], d["g"], d["beta"], h0=d.get("h0"))
    arrs = _pack(d, prec)
    arrs.update(o=np.asarray(o, np.float32), ht=np.asarray(ht, np.float32),
                meta=np.array([B, T, H, dk, seed], np.int64), prec=np.array(prec))
    np.savez_compressed(HERE / f"{name}.npz", **arrs)


def varlen_case(name, lengths, H, dk, seed, prec, h0_std):
    lengths = np.asarray(lengths, np.int64)
    T = int(lengths.sum())
    cu = inputs.cu_seqlens_from_lengths(lengths)
    d = inputs.make_inputs(1, T, H, dk, dk, seed=seed, dtype=prec, h0_std=h0_std,
                           n_states=len(lengths))
    o, ht = K.recurrent_fwd(d["q"], d["k"], d["v"], d["g"], d["beta"], h0=d["h0"], cu_seqlens=cu)
    arrs = _pack(d, prec)
    arrs.update(o=np.asarray(o, np.float32), ht=np.asarray(ht, np.float32), cu_seqlens=cu,
                meta=np.array([1, T, H, dk, seed], np.int64), prec=np.array(prec))
    np.savez_compressed(HERE / f"{name}.npz", **arrs)


def decode_case(name, B, H, dk, steps, seed, prec):
    d = inputs.make_decode_inputs(B, H, dk, dk, steps, seed=seed, dtype=prec)
    o, S = K.decode_steps(d["q"], d["k"], d["v"], d["g"], d["beta"], d["S"])
    arrs = _pack(d, prec)
    arrs.update(S0=d["S"].astype(np.float32), o=np.asarray(o, np.float32),
                S=np.asarray(S, np.float32), meta=np.array([B, H, dk, steps, seed], np.int64),
                prec=np.array(prec))
    np.savez_compressed(HERE / f"{name}.npz", **arrs)


CASES = {
    # config-0 style (fp32, d=64) with a ragged tail and two heads
    "dense_fp32_d64": lambda: dense_case("dense_fp32_d64", 1, 72, 2, 64, 1101, "fp32"),
    # bf16, d=128, nonzero initial state, T not a multiple of the chunk
    "dense_bf16_d128_h0": lambda: dense_case("dense_bf16_d128_h0", 1, 70, 1, 128, 1102, "bf16",
                                             h0_std=0.02),
    # packed varlen with an empty and a one-token sequence, per-sequence h0
    "varlen_bf16_d64": lambda: varlen_case("varlen_bf16_d64", [37, 0, 70, 1], 1, 64, 1103, "bf16",
                                           h0_std=0.02),
    # three decode steps on an N(0, 0.02^2) state
    "decode_bf16_d64": lambda: decode_case("decode_bf16_d64", 2, 2, 64, 3, 1104, "bf16"),
}


def load(name):
    """Fixture ``name`` as a dict of float32/int arrays (bf16 bits decoded to float32)."""
    z = np.load(HERE / f"{name}.npz", allow_pickle=False)
    out = {key: z[key] for key in z.files}
    prec = str(out.pop("prec"))
    if prec == "bf16":
        for key in ("q", "k", "v", "g", "beta"):
            out[key] = (out[key].astype(np.uint32) << 16).view(np.float32)
    out["prec"] = prec
    return out


if __name__ == "__main__":
    for name, make in CASES.items():
        make()
        print(f"wrote {name}.npz ({(HERE / f'{name}.npz').stat().st_size} bytes)")
