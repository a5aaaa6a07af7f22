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

// ---------------------------------------------------------------------------
// The layer's decode step fused: one workgroup of 512 threads per (b, h).
// Threads t < 3d each own one channel of q, k or v: the short conv over the
// carried buffer rows (which the thread then shifts in place), swish, and for
// q and k the head's L2 norm (a reduction over the d threads of the tensor);
// q, k, v are rounded to the input dtype as the layer's other paths hand
// them to the recurrence.  Then the step of kda_decode_kernel over the whole
// head (thread t owns columns 4 (t % NCQ) .. +3 and rows t / NCQ + RG i of the
// fp32 state, read before any of the small vectors are needed), and the
// epilogue on o by the NCQ threads that hold it: RMSNorm over the head times
// sigmoid(gate).  One launch per token instead of three, no workspace.
// ---------------------------------------------------------------------------
constexpr int kDecLayerThreads = 512;
constexpr int kMaxTaps = 8;

template <int DT>
__device__ __forceinline__ float round_to(float x) {
  if constexpr (DT == 1) return __uint_as_float(static_cast<uint32_t>(f32_to_bf16_bits(x)) << 16);
  else if constexpr (DT == 2) return static_cast<float>(static_cast<_Float16>(x));
  else return x;
}

template <int D, int DT, int OUT_DT>
__global__ __launch_bounds__(kDecLayerThreads) void kda_decode_layer_kernel(DecodeLayerArgs a) {
  constexpr int NT = kDecLayerThreads;
  constexpr int NCQ = D / 4;             // float4 column groups per state row
  constexpr int RG = NT / NCQ;           // row groups
  constexpr int RPT = D / RG;            // state rows per thread
  constexpr int WPT = D / 64;            // wavefronts per prologue tensor
  static_assert(NT % NCQ == 0 && D % RG == 0 && 3 * D <= NT && D % 64 == 0, "decode layer tiling");
  __shared__ float qs[D], ks[D], vs[D], as[D];
  __shared__ f4 red_u[RG][NCQ], red_w[RG][NCQ];
  __shared__ float red_n[NT / 64];
  __shared__ float kq_s;

  const int tid = threadIdx.x;
  const int bh = blockIdx.x;
  const int b = bh / a.H, h = bh - b * a.H;
  const int64_t HD = static_cast<int64_t>(a.H) * D;
  const int K = a.K;
  // ---- small loads first (memory operations retire in order) ----------------
  const int tt = min(tid / D, 2);        // prologue tensor of this thread (threads >= 3d: a copy of v, dropped)
  const int c = tid % D;
  const int64_t xc = static_cast<int64_t>(b) * HD + h * D + c;
  const void* xp = tt == 0 ? a.x[0] : (tt == 1 ? a.x[1] : a.x[2]);
  const float* wp = tt == 0 ? a.w[0] : (tt == 1 ? a.w[1] : a.w[2]);
  float* bp = tt == 0 ? a.buf[0] : (tt == 1 ? a.buf[1] : a.buf[2]);
  const float xv = ld1<DT>(xp, xc);
  float wt[kMaxTaps], hb[kMaxTaps - 1];
#pragma unroll
  for (int i = 0; i < kMaxTaps; ++i) {
    const float w = wp[static_cast<int64_t>(min(i, K - 1)) * HD + h * D + c];
    wt[i] = i < K ? w : 0.f;
  }
  const float* brow = bp + static_cast<int64_t>(b) * (K > 1 ? K - 1 : 1) * HD + h * D + c;
#pragma unroll
  for (int j = 0; j < kMaxTaps - 1; ++j) {
    const float v = brow[static_cast<int64_t>(max(0, min(j, K - 2))) * HD];   // a valid row; K == 1: row 0 of a stand-in
    hb[j] = j < K - 1 ? v : 0.f;
  }
  const float g_c = ld1<DT>(a.g, static_cast<int64_t>(bh) * D + (tid % D));
  const float beta = ld1<DT>(a.beta, bh);
  const int cq = tid % NCQ, rg = tid / NCQ;
  const f4 gz = ld4<DT>(a.gate, static_cast<int64_t>(b) * HD + h * D + 4 * cq);
  __builtin_amdgcn_sched_barrier(0);     // keep the small loads ahead of the state read
  float* S = a.state + static_cast<int64_t>(bh) * D * D;
  f4 sv[RPT];
#pragma unroll
  for (int i = 0; i < RPT; ++i)
    sv[i] = __builtin_nontemporal_load(reinterpret_cast<const f4*>(S + static_cast<int64_t>(rg + RG * i) * D) + cq);

  // ---- prologue ----------------------------------------------------------------
  // a = w[0] x_t + sum_{i >= 1} w[i] x_{t-i}, x_{t-i} = buffer row K-1-i
  float acc = wt[0] * xv;
#pragma unroll
  for (int i = 1; i < kMaxTaps; ++i) {
    const int j = K - 1 - i;             // buffer row of x_{t-i} (taps past K are zero)
    float hv = 0.f;
#pragma unroll
    for (int jj = 0; jj < kMaxTaps - 1; ++jj) hv = (jj == j) ? hb[jj] : hv;
    acc = fmaf(wt[i], hv, acc);
  }
  const float sw = acc * sigmoid_f32(acc);
  if (tid < 3 * D && K > 1) {            // the buffer shifts by one row: rows 1.. move up, x_t enters last
    float* bw = bp + static_cast<int64_t>(b) * (K - 1) * HD + h * D + c;
#pragma unroll
    for (int j = 0; j < kMaxTaps - 1; ++j) {
      if (j >= K - 1) break;
      bw[static_cast<int64_t>(j) * HD] = (j + 1 < K - 1) ? hb[j + 1] : xv;
    }
  }
  // head L2 norm of q and k: a sum over the d threads of the tensor
  float ss = sw * sw;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, 64);
  if ((tid & 63) == 0) red_n[tid >> 6] = ss;
  if (tid < D) as[tid] = fast_exp2(g_c * kLog2e);
  __syncthreads();
  if (tid < 3 * D) {
    float val = sw;
    if (tt < 2) {
      float tot = 0.f;
#pragma unroll
      for (int w = 0; w < WPT; ++w) tot += red_n[tt * WPT + w];
      val = sw / (__builtin_amdgcn_sqrtf(tot) + 1e-12f);
    }
    val = round_to<DT>(val);
    if (tt == 0) qs[c] = val * a.scale;
    else if (tt == 1) ks[c] = val;
    else vs[c] = val;
  }
  __syncthreads();
  // ---- recurrence: S~ = diag(alpha) S, u = S~^T k, S' = S~ + beta k (v - u)^T,
  //      o = S~^T q + beta (v - u) (k . q)
  if (tid < 64) {
    float p = 0.f;
    for (int d = tid; d < D; d += 64) p += ks[d] * qs[d];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) p += __shfl_xor(p, off, 64);
    if (tid == 0) kq_s = p;
  }
  f4 pu = {0, 0, 0, 0}, pw = {0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int d = rg + RG * i;
    sv[i] *= as[d];
    pu += ks[d] * sv[i];
    pw += qs[d] * sv[i];
  }
  red_u[rg][cq] = pu;
  red_w[rg][cq] = pw;
  __syncthreads();
  f4 uu = {0, 0, 0, 0}, ww = {0, 0, 0, 0};
#pragma unroll
  for (int g = 0; g < RG; ++g) { uu += red_u[g][cq]; ww += red_w[g][cq]; }
  const f4 vv = {vs[4 * cq], vs[4 * cq + 1], vs[4 * cq + 2], vs[4 * cq + 3]};
  const f4 delta = beta * (vv - uu);
  const float kq = kq_s;
#pragma unroll
  for (int i = 0; i < RPT; ++i) {
    const int d = rg + RG * i;
    __builtin_nontemporal_store(sv[i] + ks[d] * delta, reinterpret_cast<f4*>(S + static_cast<int64_t>(d) * D) + cq);
  }
  // ---- epilogue: y = sigmoid(gate) o / sqrt(mean(o^2) + eps), threads rg == 0 ----
  if (rg == 0) {
    const f4 o = ww + kq * delta;
    float so = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) so = fmaf(o[e], o[e], so);
#pragma unroll
    for (int off = NCQ / 2; off >= 1; off >>= 1) so += __shfl_xor(so, off, 64);
    const float rr = __builtin_amdgcn_rsqf(so * (1.f / D) + a.eps);
    f4 y;
#pragma unroll
    for (int e = 0; e < 4; ++e) y[e] = sigmoid_f32(gz[e]) * o[e] * rr;
    const int64_t yi = static_cast<int64_t>(b) * HD + h * D + 4 * cq;
    if constexpr (OUT_DT == 0) {
      *reinterpret_cast<f4*>(static_cast<float*>(a.y) + yi) = y;
    } else {
      uint2 pk;
      pk.x = static_cast<uint32_t>(f32_to_bf16_bits(y[0])) | (static_cast<uint32_t>(f32_to_bf16_bits(y[1])) << 16);
      pk.y = static_cast<uint32_t>(f32_to_bf16_bits(y[2])) | (static_cast<uint32_t>(f32_to_bf16_bits(y[3])) << 16);
      *reinterpret_cast<uint2*>(static_cast<u16*>(a.y) + yi) = pk;
    }
  }
}

hipError_t launch_decode_layer(const DecodeLayerArgs& a, int d, int dt, int out_dt, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(a.B * a.H)), blk(kDecLayerThreads);
#define KDA_DL(D_, T_, O_) \
  if (d == D_ && dt == T_ && out_dt == O_) { \
    hipLaunchKernelGGL((kda_decode_layer_kernel<D_, T_, O_>), grid, blk, 0, s, a); \
    return hipGetLastError(); \
  }
  KDA_DL(128, 0, 0) KDA_DL(128, 1, 0) KDA_DL(128, 0, 1) KDA_DL(128, 1, 1)
  KDA_DL(64, 0, 0) KDA_DL(64, 1, 0) KDA_DL(64, 0, 1) KDA_DL(64, 1, 1)
#undef KDA_DL
  return hipErrorInvalidValue;
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
