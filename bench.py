#!/usr/bin/env python
"""Benchmark of the MI355X KDA hot path (one GPU).

Headline (the ``value``): chunked KDA forward throughput in tokens/s at
B=4, T=4096, H=16, dk=dv=128, C=64, bf16 inputs, fp32 o and fp32 final state
(``configs[1]`` of the benchmark definition), inputs resident in HBM.  One
"step" = one ``kda_chunk_fwd`` over the whole batch into preallocated o and
final-state buffers.  Before the ``--warmup`` steps, a fixed clock ramp of
``CLOCK_RAMP_CALLS`` untimed calls runs whatever ``--warmup`` is: after idle
the GPU's clocks ramp up over the first ~80 calls (336 us per call for the
first 20, 244 us from the 80th on), and the timed steps are meant to see the
steady state.  The JSON line reports the ramp as ``clock_ramp_calls``.

Also reported on the same JSON line:
* TFLOP/s and % of bf16 dense MFMA peak with the algorithmic count
  ``8*C*d + 6*d^2`` FLOP per token-head;
* ``roofline``: algorithmic bytes (read q, k, v, g, beta; write o fp32 and the
  final state fp32 = 407.4 MB) over the average duration of one forward call
  (its two kernels), measured with HIP events on the stream they are launched
  on; ``traffic`` is the HBM bytes per call measured by rocprofv3
  (FETCH_SIZE + WRITE_SIZE, calibrated), read from the committed summary
  under ``profiles/``;
* ``decode``: the recurrent decode step at B=256, H=16, d=128 (fp32 state
  read-modified-written in place, bf16 inputs), iterated 128 steps, as GB/s
  against the 8 TB/s HBM peak (``configs[4]``);
* ``backward``: the chunked backward (``kda_chunk_bwd``: dq, dk, dv, dg,
  dbeta, dh0 from fp32 do and dht) on the same config-1 inputs, per call, with
  its algorithmic bytes (read q, k, v, g, beta bf16 and do fp32 plus dht;
  write the five gradients and dh0 fp32) against the HBM peak;
* ``layer``: the chunked layer forward ``kda_layer_fwd`` (short conv, swish
  and L2 norm fused into the intra kernel, the scan, the RMSNorm x sigmoid
  gate epilogue) on config-1 shapes with K = 4, bf16 projections and output;
* ``layer_backward``: the layer's backward on the same shapes -- the
  prologue and epilogue adjoints (``kda_prologue_bwd``, ``kda_epilogue_bwd``)
  per call against their algorithmic bytes, and the whole backward of
  ``kda_layer`` (q, k, v and o recomputed, then epilogue, chunked and
  prologue backward);
* ``decode_layer``: the layer decode step (prologue, recurrent step,
  epilogue) per token, eager against a HIP graph of 64 tokens, at B=1 and
  B=256;
* ``cc_scan_seam``: the reference's seam ``cc_scan`` and its backward rule
  ``cc_scan_bwd`` on one batch element of config 1 (alpha / beta32 operands,
  the reference's call shape), per call, and (``batched``) on the whole
  batch in one call with a leading batch axis;
* ``config2``, ``config3``: the chunked forward at ``configs[2]`` (B=1,
  T=65536: 1 024 serial chunks per chain) and ``configs[3]`` (64 sequences
  of U[128, 8192] tokens packed with cu_seqlens, h0 and final state per
  sequence), each per call with its own ``roofline`` over its algorithmic
  bytes;
* ``ut_solve``: the standalone unit-triangular solve at the reference's case
  (H=12, C=64, N=dk+dv=256, fp32), both orientations, per call;
* ``copy_gbps_measured`` and ``gemm_bf16_tflops_measured``: the box's own
  ceilings beside the datasheet peaks (a 1 GiB device copy; a contiguous
  8192^3 bf16 ``torch.mm``, fp32 accumulate);
* ``cpu_baseline``: the oracle's fp32 restatement of the reference jax body
  (torch CPU, all available cores) timed on a bounded sample of the same
  workload on this host.

``--gpus N`` with N > 1 exits: this build measures one GPU.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time

import torch

HBM_PEAK_GBPS = 8000.0
TRAFFIC_PROFILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                               "kda_fwd_decode_config1_config4_hbm_traffic.md")
MFMA_BF16_PEAK_TFLOPS = 2516.6

CFG = dict(B=4, T=4096, H=16, dk=128, dv=128, C=64)
# untimed forward calls before the warm-up proper (clock ramp after idle)
CLOCK_RAMP_CALLS = 150


def flops_per_token_head(C, d):
    return 8 * C * d + 6 * d * d


def reference_cost_flops_per_token_head(C, dk, dv, tile=16):
    """The reference's executed-work convention, ``cost()`` of
    ``net/kernels/kda_cc_fused_persist.py:298-318``, per token-head: the chunk's
    score matrices, their tile-wise rebuild, the solve's right-hand side and
    power chain, w·S / inter, intra and the state update, divided by C.
    344,064 at C = 64, d = 128, tile = 16."""
    ntile = -(-C // tile)
    per_chunk = (4 * C * C * dk + 4 * ntile * C * C * dk + 4 * C * C * (dk + dv)
                 + 2 * C * (dk + dv) * dk + 2 * C * dv * C + 2 * dk * dv * C)
    return per_chunk // C


def fwd_bytes(B, T, H, dk, dv, in_bytes=2, o_bytes=4):
    n = B * T * H
    return n * (3 * dk + dv) * in_bytes + n * in_bytes + n * dv * o_bytes + B * H * dk * dv * 4


def decode_bytes(B, H, dk, dv, in_bytes=2, o_bytes=4):
    n = B * H
    return 2 * n * dk * dv * 4 + n * (3 * dk + dv + 1) * in_bytes + n * dv * o_bytes


def measured_traffic(key):
    """HBM bytes per call from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
    summary (calibrated against a device copy of known size), or None."""
    try:
        with open(TRAFFIC_PROFILE) as f:
            for line in f:
                if line.startswith(key + ":"):
                    return int(line.split(":", 1)[1])
    except (OSError, ValueError):
        pass
    return None


def make_inputs_gpu(B, T, H, dk, dv, seed, device, dtype=torch.bfloat16):
    """Config distributions on the GPU: q,k = l2norm(N(0,1)); v ~ N(0,1);
    beta = sigmoid(N(0,1)); g = -softplus(N(0,1)) * exp(a_h), a_h ~ U(-2,0)."""
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)

    def l2n(x):
        return x / (x.norm(dim=-1, keepdim=True) + 1e-12)

    q = l2n(torch.randn(B, T, H, dk, device=device, generator=gen)).to(dtype)
    k = l2n(torch.randn(B, T, H, dk, device=device, generator=gen)).to(dtype)
    v = torch.randn(B, T, H, dv, device=device, generator=gen).to(dtype)
    beta = torch.sigmoid(torch.randn(B, T, H, device=device, generator=gen)).to(dtype)
    gz = torch.randn(B, T, H, dk, device=device, generator=gen)
    a = torch.rand(H, device=device, generator=gen) * -2.0
    g = (-torch.nn.functional.softplus(gz) * torch.exp(a)[None, None, :, None]).to(dtype)
    return q, k, v, g, beta


def gemm_bf16_tflops(device, n=8192, reps=10):
    """Dense bf16 matrix-core rate the box reaches through the vendor GEMM
    (torch.mm, contiguous n x n operands, fp32 accumulate): the practical
    ceiling next to the 2 516.6 TFLOP/s datasheet peak."""
    gen = torch.Generator(device=device)
    gen.manual_seed(7)
    a = torch.randn(n, n, device=device, generator=gen).to(torch.bfloat16)
    b = torch.randn(n, n, device=device, generator=gen).to(torch.bfloat16)
    for _ in range(3):
        torch.mm(a, b)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        torch.mm(a, b)
    e1.record()
    torch.cuda.synchronize()
    t = e0.elapsed_time(e1) / 1e3 / reps
    return 2.0 * n ** 3 / t / 1e12


def copy_bandwidth(device, nbytes=1 << 30, reps=10):
    x = torch.empty(nbytes // 4, dtype=torch.float32, device=device)
    y = torch.empty_like(x)
    y.copy_(x)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        y.copy_(x)
    e1.record()
    torch.cuda.synchronize()
    t = e0.elapsed_time(e1) / 1e3 / reps
    return 2 * nbytes / t / 1e9


def bench_forward(args, device):
    import axiom_amd
    from axiom_amd import kda as kmod
    B, T, H, dk, dv, C = (CFG[k] for k in ("B", "T", "H", "dk", "dv", "C"))
    q, k, v, g, beta = make_inputs_gpu(B, T, H, dk, dv, args.seed, device)
    ws = torch.empty(kmod.chunk_fwd_workspace_bytes(B, T, H, dk, dv), dtype=torch.uint8, device=device)
    o = torch.empty(B, T, H, dv, dtype=torch.float32, device=device)
    ht = torch.empty(B, H, dk, dv, dtype=torch.float32, device=device)

    def call():
        return axiom_amd.kda_chunk_fwd(q, k, v, g, beta, workspace=ws, out=o, final_state=ht)

    # clock ramp: after idle the GPU's clocks take ~80 calls to reach steady
    # state; these calls are untimed and independent of --warmup
    for _ in range(CLOCK_RAMP_CALLS):
        call()
    for _ in range(args.warmup):
        call()
    torch.cuda.synchronize()
    # the timed steps: nothing but the calls between the two synchronisations
    t0 = time.perf_counter()
    for _ in range(args.steps):
        call()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    # per-call durations from HIP events on the stream the kernels run on, in
    # a second pass of the same calls (an event record between calls costs
    # GPU time of its own, so it stays out of the timed steps)
    stream = torch.cuda.current_stream(device)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(args.steps)]
    for i in range(args.steps):
        ev[i][0].record(stream)
        call()
        ev[i][1].record(stream)
    torch.cuda.synchronize()
    per_launch = [a.elapsed_time(b) / 1e3 for a, b in ev]
    return dict(wall=wall, per_launch=per_launch, o=o, ht=ht, inputs=(q, k, v, g, beta))


def bench_decode(args, device):
    import axiom_amd
    B, H, d, steps = 256, 16, 128, args.decode_steps
    gen = torch.Generator(device=device)
    gen.manual_seed(args.seed + 1)
    q, k, v, g, beta = make_inputs_gpu(steps, B, H, d, d, args.seed + 2, device)
    S = torch.randn(B, H, d, d, device=device, generator=gen) * 0.02
    stream = torch.cuda.current_stream(device)
    for t in range(min(8, steps)):                       # warm-up on a scratch copy
        axiom_amd.kda_recurrent_step(q[t], k[t], v[t], g[t], beta[t], S.clone())
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for t in range(steps):
        axiom_amd.kda_recurrent_step(q[t], k[t], v[t], g[t], beta[t], S)
    e1.record(stream)
    torch.cuda.synchronize()
    t_step = e0.elapsed_time(e1) / 1e3 / steps
    nbytes = decode_bytes(B, H, d, d)
    gbps = nbytes / t_step / 1e9
    return dict(us_per_step=t_step * 1e6, gbps=gbps, frac=gbps / HBM_PEAK_GBPS,
                bytes_per_step=nbytes, traffic=measured_traffic("decode_traffic_bytes_per_step"),
                steps=steps, config="B256 H16 d128 bf16, fp32 state in place")


def bwd_bytes(B, T, H, dk, dv, in_bytes=2):
    n = B * T * H
    read = n * ((3 * dk + dv) * in_bytes + in_bytes + dv * 4) + B * H * dk * dv * 4
    write = n * ((3 * dk + dv) * 4 + 4) + B * H * dk * dv * 4
    return read + write


def bench_backward(args, fwd_inputs, device):
    import axiom_amd
    from axiom_amd import kda as kmod
    q, k, v, g, beta = fwd_inputs
    B, T, H, dk = q.shape
    dv = v.shape[3]
    gen = torch.Generator(device=device)
    gen.manual_seed(args.seed + 3)
    do = torch.randn(B, T, H, dv, device=device, generator=gen)
    dht = torch.randn(B, H, dk, dv, device=device, generator=gen) * 0.1
    ws = torch.empty(kmod.chunk_bwd_workspace_bytes(B, T, H, dk, dv), dtype=torch.uint8, device=device)
    stream = torch.cuda.current_stream(device)
    for _ in range(5):
        axiom_amd.kda_chunk_bwd(q, k, v, g, beta, do, dht=dht, workspace=ws)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(args.bwd_steps):
        axiom_amd.kda_chunk_bwd(q, k, v, g, beta, do, dht=dht, workspace=ws)
    e1.record(stream)
    torch.cuda.synchronize()
    t_call = e0.elapsed_time(e1) / 1e3 / args.bwd_steps
    nbytes = bwd_bytes(B, T, H, dk, dv)
    gbps = nbytes / t_call / 1e9
    return dict(us_per_call=t_call * 1e6, tokens_per_s=B * T / t_call, calls=args.bwd_steps,
                roofline={"bound": "hbm", "achieved": gbps, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                          "frac": gbps / HBM_PEAK_GBPS, "algorithmic_bytes_per_call": nbytes,
                          "traffic": measured_traffic("backward_traffic_bytes_per_call")},
                kernels="kda_bwd_prep + kda_bwd_fscan16 + kda_bwd_rscan16 + kda_bwd_chunk (fp16 forward-side "
                        "workspace, fp32 cotangents; fp16 and bf16 hi/lo products)",
                config="B4 T4096 H16 d128 bf16 inputs, fp32 do and dht, zero h0")


def bench_decode_layer(args, device):
    """Layer decode steps (prologue, recurrent step, epilogue; conv buffers and
    state in place) per token: eager launches against one HIP graph replaying
    64 tokens, at B=1 (launch-bound serving) and B=256 (configs[4]'s batch)."""
    import axiom_amd
    H, d, K, steps = 16, 128, 4, 64
    out = {}
    stream = torch.cuda.current_stream(device)
    for B in (1, 256):
        gen = torch.Generator(device=device)
        gen.manual_seed(args.seed + 8)
        bf = torch.bfloat16
        toks = [[torch.randn(B, H * d, device=device, generator=gen).to(bf) for _ in range(4)] for _ in range(steps)]
        gs = [(-torch.nn.functional.softplus(torch.randn(B, H, d, device=device, generator=gen))).to(bf)
              for _ in range(steps)]
        bs = [torch.sigmoid(torch.randn(B, H, device=device, generator=gen)).to(bf) for _ in range(steps)]
        ws_ = [torch.randn(K, H * d, device=device, generator=gen) * 0.4 for _ in range(3)]
        state = torch.randn(B, H, d, d, device=device, generator=gen) * 0.02
        bufs = [torch.zeros(B, K - 1, H * d, device=device) for _ in range(3)]

        def run():
            return [axiom_amd.kda_decode_layer_step(qp, kp, vp, gs[t], bs[t], gt, *ws_, bufs, state)
                    for t, (qp, kp, vp, gt) in enumerate(toks)]

        run()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        run()
        e1.record(stream)
        torch.cuda.synchronize()
        t_eager = e0.elapsed_time(e1) / 1e3 / steps
        side = torch.cuda.Stream()
        side.wait_stream(stream)
        with torch.cuda.stream(side):
            run()
        stream.wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            run()
        graph.replay()
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(5):
            graph.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        t_graph = e0.elapsed_time(e1) / 1e3 / (5 * steps)
        out[f"B{B}"] = dict(us_per_token_eager=t_eager * 1e6, us_per_token_graph=t_graph * 1e6)
    out["config"] = "H16 d128 K4 bf16, 64 tokens per graph"
    return out


def layer_bytes(B, T, H, d, K):
    """Read qp, kp, vp, g, gate bf16, beta bf16, conv taps fp32; write y bf16 and hT fp32."""
    n = B * T * H
    return n * d * 5 * 2 + n * 2 + 3 * K * H * d * 4 + n * d * 2 + B * H * d * d * 4


def bench_layer(args, fwd_inputs, device):
    """The chunked layer forward (prologue fused into the intra kernel, scan, epilogue)."""
    import axiom_amd
    from axiom_amd import kda as kmod
    q, k, v, g, beta = fwd_inputs
    B, T, H, d = q.shape
    K = 4
    gen = torch.Generator(device=device)
    gen.manual_seed(args.seed + 5)
    xs = [torch.randn(B, T, H * d, device=device, generator=gen).to(torch.bfloat16) for _ in range(3)]
    ws_ = [torch.randn(K, H * d, device=device, generator=gen) * 0.4 for _ in range(3)]
    gate = torch.randn(B, T, H * d, device=device, generator=gen).to(torch.bfloat16)
    ws = torch.empty(kmod.layer_fwd_workspace_bytes(B, T, H, d, K), dtype=torch.uint8, device=device)
    stream = torch.cuda.current_stream(device)

    cws = torch.empty(kmod.chunk_fwd_workspace_bytes(B, T, H, d, d), dtype=torch.uint8, device=device)

    def call():
        return axiom_amd.kda_layer_fwd(*xs, g, beta, gate, *ws_, out_dtype=torch.bfloat16,
                                       return_conv_state=False, workspace=ws)

    def unfused():   # the same layer as three entry points (q, k, v and o through memory)
        qq, kk, vv, _ = axiom_amd.kda_prologue(*xs, *ws_, H, out_dtype=torch.bfloat16, return_state=False)
        o, _ = axiom_amd.kda_chunk_fwd(qq, kk, vv, g, beta, workspace=cws)
        return axiom_amd.kda_epilogue(o, gate, out_dtype=torch.bfloat16)

    def timed(f):
        for _ in range(5):
            f()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(args.steps):
            f()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / 1e3 / args.steps
    t_call = timed(call)
    t_unfused = timed(unfused)
    nbytes = layer_bytes(B, T, H, d, K)
    gbps = nbytes / t_call / 1e9
    return dict(us_per_call=t_call * 1e6, tokens_per_s=B * T / t_call, unfused_us_per_call=t_unfused * 1e6,
                roofline={"bound": "hbm", "achieved": gbps, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                          "frac": gbps / HBM_PEAK_GBPS, "algorithmic_bytes_per_call": nbytes},
                kernels="kda_intra_kernel with the fused short conv + kda_state_col_kernel + kda_epilogue_kernel",
                config="B4 T4096 H16 d128 K4, bf16 projections, gates and y, fp32 o inside, zero h0")


def bench_layer_bwd(args, fwd_inputs, device):
    """The layer backward at config-1 shapes (K = 4, bf16 projections, gate and
    dy): the prologue and epilogue adjoints on their own, and the whole
    backward of ``kda_layer`` (q, k, v recomputed, o kept by the forward;
    epilogue backward, chunked backward, prologue backward)."""
    import axiom_amd
    from axiom_amd import kda as kmod
    q, k, v, g, beta = fwd_inputs
    B, T, H, d = q.shape
    K = 4
    gen = torch.Generator(device=device)
    gen.manual_seed(args.seed + 7)
    bf = torch.bfloat16
    xs = [torch.randn(B, T, H * d, device=device, generator=gen).to(bf) for _ in range(3)]
    ws_ = [torch.randn(K, H * d, device=device, generator=gen) * 0.4 for _ in range(3)]
    gate = torch.randn(B, T, H * d, device=device, generator=gen).to(bf)
    dy = torch.randn(B, T, H * d, device=device, generator=gen).to(bf)
    dqkv = [torch.randn(B, T, H, d, device=device, generator=gen) for _ in range(3)]
    o = torch.randn(B, T, H, d, device=device, generator=gen)
    pws = torch.empty(kmod.prologue_bwd_workspace_bytes(B, T, H, d, K), dtype=torch.uint8, device=device)
    bws = torch.empty(kmod.chunk_bwd_workspace_bytes(B, T, H, d, d), dtype=torch.uint8, device=device)
    stream = torch.cuda.current_stream(device)

    def timed(f, steps):
        for _ in range(3):
            f()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            f()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / 1e3 / steps

    def whole():   # the forward kept o (kda_layer_fwd's o_out): q, k, v are recomputed
        qq, kk, vv, _ = axiom_amd.kda_prologue(*xs, *ws_, H, out_dtype=bf, return_state=False)
        do, _ = axiom_amd.kda_epilogue_bwd(o, gate, dy)
        dq, dk, dv, _, _, _ = axiom_amd.kda_chunk_bwd(qq, kk, vv, g, beta, do, need_dh0=False, workspace=bws)
        return axiom_amd.kda_prologue_bwd(*xs, *ws_, dq, dk, dv, workspace=pws)

    nd = B * T * H * d
    t_pro = timed(lambda: axiom_amd.kda_prologue_bwd(*xs, *ws_, *dqkv, workspace=pws), args.steps)
    t_epi = timed(lambda: axiom_amd.kda_epilogue_bwd(o, gate, dy), args.steps)
    t_all = timed(whole, args.bwd_steps)
    pro_bytes = 3 * nd * (2 + 4 + 4) + 6 * K * H * d * 4     # x bf16, dq/dk/dv fp32 in; dx fp32, taps, dw
    epi_bytes = nd * (4 + 2 + 2 + 4 + 2)                    # o fp32, gate, dy bf16 in; do fp32, dgate bf16
    return dict(
        prologue_bwd={"us_per_call": t_pro * 1e6, "algorithmic_bytes": pro_bytes,
                      "gbps": pro_bytes / t_pro / 1e9, "frac": pro_bytes / t_pro / 1e9 / HBM_PEAK_GBPS,
                      "kernels": "kda_prologue_bwd_kernel (one pass) + kda_prologue_bwd_dw_kernel"},
        epilogue_bwd={"us_per_call": t_epi * 1e6, "algorithmic_bytes": epi_bytes,
                      "gbps": epi_bytes / t_epi / 1e9, "frac": epi_bytes / t_epi / 1e9 / HBM_PEAK_GBPS},
        layer_bwd_us_per_call=t_all * 1e6, layer_bwd_tokens_per_s=B * T / t_all,
        config="B4 T4096 H16 d128 K4, bf16 projections, gate and dy; the whole backward recomputes q, k, v "
               "(o kept by the forward)")


def bench_cc_scan(args, fwd_inputs, device):
    """The reference's own seam (``cc_scan`` and its backward rule) on one batch
    element of config 1 -- how the reference calls it, vmapped over B -- with
    the alpha / beta32 operands: the adapter (g = log alpha, beta = mean of the
    32 columns) plus the dense kernels."""
    import axiom_amd
    q, k, v, g, beta = fwd_inputs
    _, T, H, d = q.shape
    q2, k2, v2 = (x[0].reshape(T, H * d).contiguous() for x in (q, k, v))
    alpha = torch.exp(g[0].float()).reshape(T, H * d).contiguous()
    beta32 = beta[0].float().reshape(T, H, 1).expand(T, H, 32).reshape(T, H * 32).contiguous()
    S = torch.zeros(H, d, d, device=device)
    gen = torch.Generator(device=device)
    gen.manual_seed(args.seed + 9)
    do = torch.randn(T, H * d, device=device, generator=gen)
    dS = torch.randn(H, d, d, device=device, generator=gen) * 0.1
    stream = torch.cuda.current_stream(device)

    def timed(f, steps):
        for _ in range(3):
            f()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            f()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / 1e3 / steps
    t_f = timed(lambda: axiom_amd.cc_scan(q2, k2, v2, alpha, beta32, S, tile=16, chunk=64), args.steps)
    t_b = timed(lambda: axiom_amd.cc_scan_bwd(q2, k2, v2, alpha, beta32, S, do, dS, tile=16, chunk=64),
                args.bwd_steps)
    # the whole batch in one call (the vmapped caller's form)
    B = q.shape[0]
    qb, kb, vb = (x.reshape(B, T, H * d) for x in (q, k, v))
    alpha_b = torch.exp(g.float()).reshape(B, T, H * d).contiguous()
    beta32_b = beta.float().reshape(B, T, H, 1).expand(B, T, H, 32).reshape(B, T, H * 32).contiguous()
    S_b = torch.zeros(B, H, d, d, device=device)
    do_b = torch.randn(B, T, H * d, device=device, generator=gen)
    dS_b = torch.randn(B, H, d, d, device=device, generator=gen) * 0.1
    t_fb = timed(lambda: axiom_amd.cc_scan(qb, kb, vb, alpha_b, beta32_b, S_b, tile=16, chunk=64), args.steps)
    t_bb = timed(lambda: axiom_amd.cc_scan_bwd(qb, kb, vb, alpha_b, beta32_b, S_b, do_b, dS_b, tile=16, chunk=64),
                 args.bwd_steps)
    return dict(fwd_us_per_call=t_f * 1e6, bwd_us_per_call=t_b * 1e6, tokens_per_s_fwd=T / t_f,
                config=f"one batch element: T{T} H{H} d{d}, bf16 q/k/v, fp32 alpha/beta32/S (cc_scan, cc_scan_bwd)",
                batched=dict(fwd_us_per_call=t_fb * 1e6, bwd_us_per_call=t_bb * 1e6,
                             tokens_per_s_fwd=B * T / t_fb,
                             config=f"whole batch in one call: B{B} T{T} H{H} d{d} (leading batch axis)"))


def bench_ut_solve(args, device):
    import axiom_amd
    H, C, N = 12, 64, 256
    gen = torch.Generator(device=device)
    gen.manual_seed(args.seed + 4)
    a = torch.eye(C, device=device) + torch.tril((torch.rand(H, C, C, device=device, generator=gen) - 0.5) * 0.5, -1)
    b = torch.randn(H, C, N, device=device, generator=gen)
    out = {}
    stream = torch.cuda.current_stream(device)
    for tr in (False, True):
        for _ in range(3):
            axiom_amd.ut_solve(a, b, transpose=tr)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(50):
            axiom_amd.ut_solve(a, b, transpose=tr)
        e1.record(stream)
        torch.cuda.synchronize()
        out["us_per_call_t" if tr else "us_per_call"] = e0.elapsed_time(e1) / 50 * 1e3
    out["config"] = "H12 C64 N256 fp32 (the reference's case)"
    return out


def _roofline(nbytes, t, traffic_key=None):
    achieved = nbytes / t / 1e9
    return {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBPS,
            "traffic": measured_traffic(traffic_key) if traffic_key else None,
            "algorithmic_bytes_per_call": nbytes}


def bench_other_configs(args, device):
    """Forward at configs 2 (B1 T65536, 1 024 serial chunks per chain) and 3
    (64 packed sequences of U[128, 8192] tokens, per-sequence h0 and final
    states): per call with HIP events on the kernels' stream, inputs resident,
    each with its algorithmic bytes (read q, k, v, g, beta; write o fp32 and
    the final states; config 3 also reads its h0) against the HBM peak."""
    import axiom_amd
    from axiom_amd import kda as kmod
    from oracle import inputs as oin
    stream = torch.cuda.current_stream(device)

    def timed(f, n):
        for _ in range(3):
            f()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(n):
            f()
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / 1e3 / n

    out = {}
    H, d = CFG["H"], CFG["dk"]
    T2 = 65536
    q, k, v, g, beta = make_inputs_gpu(1, T2, H, d, d, args.seed + 6, device)
    ws = torch.empty(kmod.chunk_fwd_workspace_bytes(1, T2, H, d, d), dtype=torch.uint8, device=device)
    o = torch.empty(1, T2, H, d, device=device)
    ht = torch.empty(1, H, d, d, device=device)
    t = timed(lambda: axiom_amd.kda_chunk_fwd(q, k, v, g, beta, workspace=ws, out=o, final_state=ht),
              args.config_calls)
    nb = fwd_bytes(1, T2, H, d, d)
    out["config2"] = dict(us_per_call=t * 1e6, tokens_per_s=T2 / t, calls=args.config_calls,
                          roofline=_roofline(nb, t, "config2_traffic_bytes_per_call"),
                          workload="B1 T65536 H16 d128 bf16, fp32 o and final state, zero initial state")
    del q, k, v, g, beta, ws, o, ht
    lengths = oin.make_varlen_lengths(64, 128, 8192, seed=3)
    cu = torch.from_numpy(oin.cu_seqlens_from_lengths(lengths)).to(device)
    T3 = int(lengths.sum())
    q, k, v, g, beta = make_inputs_gpu(1, T3, H, d, d, args.seed + 7, device)
    gen = torch.Generator(device=device)
    gen.manual_seed(args.seed + 8)
    h0 = torch.randn(len(lengths), H, d, d, device=device, generator=gen) * 0.02
    ws = torch.empty(kmod.chunk_fwd_workspace_bytes(1, T3, H, d, d, n_seqs=len(lengths)), dtype=torch.uint8,
                     device=device)
    o = torch.empty(1, T3, H, d, device=device)
    ht = torch.empty(len(lengths), H, d, d, device=device)
    t = timed(lambda: axiom_amd.kda_chunk_fwd(q, k, v, g, beta, initial_state=h0, cu_seqlens=cu, workspace=ws,
                                              out=o, final_state=ht), args.config_calls)
    nb = fwd_bytes(1, T3, H, d, d) + 2 * len(lengths) * H * d * d * 4 - H * d * d * 4
    out["config3"] = dict(us_per_call=t * 1e6, tokens_per_s=T3 / t, calls=args.config_calls,
                          roofline=_roofline(nb, t, "config3_traffic_bytes_per_call"),
                          workspace_bytes=int(ws.numel()),
                          workload=f"varlen 64 sequences U[128, 8192] (T={T3}) H16 d128 bf16, fp32 o, "
                                   "h0 and final state per sequence")
    return out


def cpu_baseline(fwd_inputs, seconds):
    """Oracle port (fp32, torch CPU) of the reference jax body on a bounded sample."""
    from oracle import kda_oracle as K
    n_threads = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    torch.set_num_threads(n_threads)
    q, k, v, g, beta = (x.float().cpu().numpy() for x in fwd_inputs)
    B, T, H = q.shape[:3]

    def run():
        t0 = time.perf_counter()
        K.chunk_fwd(q, k, v, g, beta, chunk=64, dtype=torch.float32)
        return time.perf_counter() - t0

    run()                                                 # warm-up round
    times = [run()]
    budget = time.perf_counter() + seconds
    while time.perf_counter() < budget or len(times) < 3:
        times.append(run())
    med = statistics.median(times)
    T_s = B * T
    cpu_model = platform.processor() or ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"value": T_s / med, "unit": "tokens/s", "cores": n_threads, "kind": "port",
            "sample": f"the full workload B={B} T={T} H={H} d=128 C=64 in fp32 (the bench inputs "
                      f"upcast), median of {len(times)} rounds, {med:.2f} s/round",
            "cpu_model": cpu_model}


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--decode-steps", type=int, default=128)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--bwd-steps", type=int, default=20)
    ap.add_argument("--no-backward", action="store_true")
    ap.add_argument("--no-other-configs", action="store_true",
                    help="skip the forward at configs 2 and 3")
    ap.add_argument("--config-calls", type=int, default=10,
                    help="timed calls of the forward at configs 2 and 3")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: every (batch, head) chain of this path is "
              "independent, multi-GPU sharding is described but not run here.", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    device = torch.device("cuda:0")
    B, T, H, dk, dv, C = (CFG[k] for k in ("B", "T", "H", "dk", "dv", "C"))

    fwd = bench_forward(args, device)
    steps = args.steps
    ms_per_step = fwd["wall"] / steps * 1e3
    t_launch = statistics.mean(fwd["per_launch"])
    tokens = B * T
    flops = tokens * H * flops_per_token_head(C, dk)
    nbytes = fwd_bytes(B, T, H, dk, dv)
    value = tokens / (fwd["wall"] / steps)
    tflops = flops / t_launch / 1e12
    achieved = nbytes / t_launch / 1e9
    line = {
        "metric": "KDA fwd tokens/s + TFLOP/s (% MFMA peak) at B4 T4096 H16 d128; decode HBM GB/s",
        "value": value,
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "clock_ramp_calls": CLOCK_RAMP_CALLS,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "chunked KDA forward B=4 T=4096 H=16 dk=dv=128 C=64, bf16 in, "
                               "fp32 o and final state, zero initial state",
                   "global_batch": B, "seq_len": T, "heads": H, "head_dim": dk, "chunk": C},
        "tflops": tflops,
        "mfma_peak_frac": tflops / MFMA_BF16_PEAK_TFLOPS,
        "us_per_launch": t_launch * 1e6,
        # secondary: the reference's own cost() FLOP convention over the same launch
        "reference_cost_tflops": tokens * H * reference_cost_flops_per_token_head(C, dk, dv) / t_launch / 1e12,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBPS,
                     "traffic": measured_traffic("traffic_bytes_per_call"),
                     "kernels": "kda_intra_kernel + kda_state_col_kernel (one kda_chunk_fwd)",
                     "algorithmic_bytes_per_launch": nbytes},
    }
    try:
        line["copy_gbps_measured"] = copy_bandwidth(device)
    except RuntimeError:
        line["copy_gbps_measured"] = None
    try:
        line["gemm_bf16_tflops_measured"] = gemm_bf16_tflops(device)
    except RuntimeError:
        line["gemm_bf16_tflops_measured"] = None
    if not args.no_decode:
        line["decode"] = bench_decode(args, device)
    if not args.no_backward:
        line["backward"] = bench_backward(args, fwd["inputs"], device)
    line["layer"] = bench_layer(args, fwd["inputs"], device)
    if not args.no_backward:
        line["layer_backward"] = bench_layer_bwd(args, fwd["inputs"], device)
    line["decode_layer"] = bench_decode_layer(args, device)
    line["cc_scan_seam"] = bench_cc_scan(args, fwd["inputs"], device)
    line["ut_solve"] = bench_ut_solve(args, device)
    if not args.no_other_configs:
        line.update(bench_other_configs(args, device))
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(fwd["inputs"], args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
