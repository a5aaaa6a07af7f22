// Single-token recurrent KDA step (decode), HBM-bound on the fp32 state.
//
// Restates the reference delta rule net/kda.py:298-310 (_delta_step) and the
// read-out net/kda.py:293 for one token per chain:
//   S~ = diag(alpha) S,  u = S~^T k,  S' = S~ + beta k (v - u)^T,  o = S'^T q
// with o computed as  S~^T q + beta (v - u) (k . q)  so S is read once and
// written once (in place).
//
// Two workgroups of 256 threads per (b, h), each owning half of the value
// columns for all channels (the column sums u = S~^T k and w = S~^T q need no
// data from the other half; q, k, alpha are read by both).  Thread t owns
// columns 4*(t % NCQ) .. +3 of its half and channel rows t / NCQ + RG*i; the
// column partial sums are reduced across the RG row groups through LDS.
// Half-width workgroups keep the state slice in 32 registers per thread, so
// more workgroups are resident per CU.

#include "kda_common.h"
#include "kda_internal.h"

namespace kda {

constexpr int kDecodeColSplit = 2;

template <int DK, int DV, int DT, int OUT_DT>
__global__ __launch_bounds__(256)
void kda_decode_kernel(DecodeArgs a) {
  constexpr int DVW = DV / kDecodeColSplit;  // value columns of this workgroup
  constexpr int NCQ = DVW / 4;           // float4 column groups per row
  constexpr int RG = 256 / NCQ;          // row groups
  constexpr int RPT = DK / RG;           // rows per thread
  static_assert(256 % NCQ == 0 && DK % RG == 0, "decode tiling");
  __shared__ float qs[DK], ks[DK], as[DK];
  __shared__ f4 red_u[RG][NCQ], red_w[RG][NCQ];
  __shared__ float kq_s;

  const int tid = threadIdx.x;
  const int bh = blockIdx.x / kDecodeColSplit;   // b * H + h
  const int c0 = (blockIdx.x % kDecodeColSplit) * DVW;
  const int64_t vec = static_cast<int64_t>(bh);
  // The small per-token loads (q, k, g, beta, v) are issued first and the
  // state read right after: memory operations retire in order, so waiting on
  // the small loads does not wait for the state, whose latency then overlaps
  // the exp, the barrier and the k.q reduction.  Every thread loads an
  // in-range q/k/g element; threads >= DK drop theirs.
  static_assert(DK <= 256, "one q/k/g element per thread");
  const int td = tid % DK;
  const float q_t = ld1<DT>(a.q, vec * DK + td);
  const float k_t = ld1<DT>(a.k, vec * DK + td);
  const float g_t = ld1<DT>(a.g, vec * DK + td);
  const int cq = tid % NCQ;
  const int rg = tid / NCQ;
  const float beta = ld1<DT>(a.beta, vec);
  const f4 vv = ld4<DT>(a.v, vec * DV + c0 + 4 * cq);
  __builtin_amdgcn_sched_barrier(0);  // keep the small loads ahead of the state read
  float* S = a.state + static_cast<int64_t>(bh) * DK * DV + c0;
  f4 sv[RPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int d = rg + RG * i;
    sv[i] = __builtin_nontemporal_load(reinterpret_cast<const f4*>(S + static_cast<int64_t>(d) * DV) + cq);
  }
  if (tid < DK) {
    qs[tid] = q_t * a.scale;
    ks[tid] = k_t;
    as[tid] = fast_exp2(g_t * kLog2e);
  }
  __syncthreads();
  if (tid < 64) {
    float p = 0.f;
    for (int d = tid; d < DK; d += 64) p += ks[d] * qs[d];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) p += __shfl_xor(p, off, 64);
    if (tid == 0) kq_s = p;
  }

  f4 pu = {0, 0, 0, 0}, pw = {0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int d = rg + RG * i;
    const float al = as[d];
    sv[i] *= al;                                   // S~ = diag(alpha) S
    pu += ks[d] * sv[i];
    pw += qs[d] * sv[i];
  }
  red_u[rg][cq] = pu;
  red_w[rg][cq] = pw;
  __syncthreads();
  f4 uu = {0, 0, 0, 0}, ww = {0, 0, 0, 0};
#pragma unroll
  for (int g = 0; g < RG; ++g) { uu += red_u[g][cq]; ww += red_w[g][cq]; }
  const f4 delta = beta * (vv - uu);              // beta (v - u)
  const float kq = kq_s;
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int d = rg + RG * i;
    const f4 out = sv[i] + ks[d] * delta;
    __builtin_nontemporal_store(out, reinterpret_cast<f4*>(S + static_cast<int64_t>(d) * DV) + cq);
  }
  if (rg == 0) {
    const f4 o = ww + kq * delta;
    const int64_t oi = vec * DV + c0 + 4 * cq;
    if constexpr (OUT_DT == 0) {
      *reinterpret_cast<f4*>(static_cast<float*>(a.o) + oi) = o;
    } else {
      uint2 pk;
      pk.x = static_cast<uint32_t>(f32_to_bf16_bits(o[0])) | (static_cast<uint32_t>(f32_to_bf16_bits(o[1])) << 16);
      pk.y = static_cast<uint32_t>(f32_to_bf16_bits(o[2])) | (static_cast<uint32_t>(f32_to_bf16_bits(o[3])) << 16);
      *reinterpret_cast<uint2*>(static_cast<u16*>(a.o) + oi) = pk;
    }
  }
}

template <int D, int DT, int OUT>
static hipError_t launch_decode_t(const DecodeArgs& a, int grid, hipStream_t s) {
  hipLaunchKernelGGL((kda_decode_kernel<D, D, DT, OUT>), dim3(grid * kDecodeColSplit), dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_decode(const DecodeArgs& a, int d, int dt, int out_dt, int grid, hipStream_t s) {
#define KDA_DEC(D, T, O) if (d == D && dt == T && out_dt == O) return launch_decode_t<D, T, O>(a, grid, s);
  KDA_DEC(128, 0, 0) KDA_DEC(128, 1, 0) KDA_DEC(128, 2, 0)
  KDA_DEC(128, 0, 1) KDA_DEC(128, 1, 1) KDA_DEC(128, 2, 1)
  KDA_DEC(64, 0, 0) KDA_DEC(64, 1, 0) KDA_DEC(64, 2, 0)
  KDA_DEC(64, 0, 1) KDA_DEC(64, 1, 1) KDA_DEC(64, 2, 1)
#undef KDA_DEC
  return hipErrorInvalidValue;
}

}  // namespace kda
