"""CPU oracle for the KDA hot path (chunked WY/UT forward, recurrent decode, varlen).

TEST INFRASTRUCTURE ONLY.  Nothing in the product package ``axiom_amd`` imports,
links or runs anything from here.  The only permitted users are ``tests/``,
``__graft_entry__.smoke()`` (as the checker of one small run) and the
``cpu_baseline`` leg of ``bench.py`` (as the timed CPU port of the reference's
jax body).  The product path raises when its HIP library is missing; it never
falls back to this package.

Modules:

* :mod:`oracle.kda_oracle` -- the restatement.  Every function cites the
  reference file:line it follows (reference = romannekrasovaillm/axiom).
* :mod:`oracle.inputs` -- the seeded input generator of the benchmark configs.
* :mod:`oracle.layer` -- the layer's prologue (short conv, swish, L2 norm) and
  epilogue (head-wise RMS norm times the sigmoid gate) and their adjoints.
* :mod:`oracle.emulate` -- the chunk body with the HIP kernels' rounding
  points (fp16 / bf16 hi-lo operands, fp32 accumulation): the error the
  kernels' operand precisions cost.

Pinning status of each function is listed in the header of
:mod:`oracle.kda_oracle`.
"""
