"""axiom_amd -- MI355X-native (gfx950) KDA hot path.

Chunked Kimi-Delta-Attention forward in WY/UT form, the single-token recurrent
decode step, varlen scheduling, the chunked backward and the layer's prologue/epilogue
(forward and backward), as hand-written HIP
kernels behind the C ABI of ``include/kda_mi355x.h``.  The Python layer (:mod:`axiom_amd.kda`) only
validates arguments and hands device pointers to that library.
"""

from .kda import (cc_scan, cc_scan_bwd, kda_chunk, kda_chunk_bwd, kda_chunk_fwd, kda_decode_layer_step,  # noqa: F401
                  kda_epilogue, kda_epilogue_bwd, kda_layer, kda_layer_fwd, kda_prologue, kda_prologue_bwd,
                  kda_recurrent_step, solve, solve_t, ut_solve, ut_solve_bwd, varlen_status)

__all__ = ["cc_scan", "cc_scan_bwd", "kda_chunk", "kda_chunk_bwd", "kda_chunk_fwd", "kda_decode_layer_step", "kda_epilogue",
           "kda_epilogue_bwd", "kda_layer", "kda_layer_fwd", "kda_prologue", "kda_prologue_bwd",
           "kda_recurrent_step", "solve", "solve_t", "ut_solve", "ut_solve_bwd", "varlen_status"]
