"""The bench line's FLOP and byte bookkeeping at config 1 (CPU).

The figures are checked against numbers computed independently of the
formulas: the reference's ``cost()`` (``net/kernels/kda_cc_fused_persist.py:298-318``)
evaluates to 344,064 FLOP per token-head at C = 64, d = 128, tile = 16; the
algorithmic forward bytes of B4 T4096 H16 d128 are q, k, v (bf16), beta
(bf16), o (fp32) and the fp32 final state, summed by hand below.
"""

from __future__ import annotations

import bench


def test_reference_cost_convention():
    assert bench.reference_cost_flops_per_token_head(64, 128, 128, tile=16) == 344_064
    # one tile spanning the chunk: the rebuild term shrinks to a single pass
    assert bench.reference_cost_flops_per_token_head(64, 128, 128, tile=64) == 344_064 - 3 * 4 * 64 * 128


def test_algorithmic_flops_and_bytes_config1():
    assert bench.flops_per_token_head(64, 128) == 163_840
    n = 4 * 4096 * 16
    by_hand = n * 512 * 2 + n * 2 + n * 128 * 4 + 4 * 16 * 128 * 128 * 4
    assert by_hand == 407_371_776
    assert bench.fwd_bytes(4, 4096, 16, 128, 128) == by_hand
