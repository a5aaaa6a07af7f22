// KDA prologue and epilogue around the chunked kernels (fp32 arithmetic).
//
// Prologue (net/kda.py:194-202 _postprocess after net/shortconv.py:14-33
// short_conv): per channel a causal depthwise convolution of the projections
// qp, kp, vp with K taps (out[t] = sum_i w[i] x[t-i], history from the conv
// buffers of a previous segment or zero), then swish (x * sigmoid(x),
// net/norm.py:15-17), then for q and k the per-head L2 normalisation
// x / (||x|| + 1e-12) (net/norm.py:53-66); outputs in the [B,T,H,d] layout
// kda_chunk_fwd takes.  The conv buffers then hold the last K-1 inputs
// (net/kda.py:383-389 _short_conv_chunk).
// Epilogue (net/kda.py:205-214 _output_gate without the W_o projection):
// y = sigmoid(gate) * o / sqrt(mean_head(o^2) + eps) (net/norm.py:69-73).
//
// One wavefront per (tensor, b, t, h) row: lane l holds channels PL*l ..
// PL*l + PL-1 (PL = d/64), the head's sum of squares is a wavefront xor-
// butterfly.  The fused prologue of the intra kernel (kda_chunk.hip) uses the
// same channel mapping, tap order and reduction order, so its q, k, v equal
// this kernel's bit for bit.  The K input rows a convolution reads are
// neighbouring rows of the same tensor (cache hits).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "kda_common.h"
#include "kda_internal.h"

namespace kda {
namespace {

constexpr int kRowsPerBlock = 4;   // wavefronts per workgroup

template <int DT>
__device__ __forceinline__ float pl_ld(const void* p, int64_t i) {
  if constexpr (DT == 0) return static_cast<const float*>(p)[i];
  else return bf16_to_f32(static_cast<const u16*>(p)[i]);
}

template <int DT>
__device__ __forceinline__ void pl_st(void* p, int64_t i, float v) {
  if constexpr (DT == 0) static_cast<float*>(p)[i] = v;
  else static_cast<u16*>(p)[i] = f32_to_bf16_bits(v);
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off, 64);
  return x;
}

template <int DI, int DO, int D>
__global__ __launch_bounds__(64 * kRowsPerBlock) void kda_prologue_kernel(PrologueArgs a) {
  constexpr int PL = D / 64;   // channels per lane
  const int lane = threadIdx.x & 63;
  const int64_t rows = static_cast<int64_t>(a.B) * a.T * a.H;
  const int64_t r = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
  if (r >= 3 * rows) return;                       // uniform per wavefront
  const int tensor = static_cast<int>(r / rows);   // 0 q, 1 k, 2 v
  const int64_t rr = r - tensor * rows;
  const int h = static_cast<int>(rr % a.H);
  const int64_t bt = rr / a.H;
  const int t = static_cast<int>(bt % a.T);
  const int b = static_cast<int>(bt / a.T);
  const void* x = tensor == 0 ? a.qp : tensor == 1 ? a.kp : a.vp;
  const float* w = tensor == 0 ? a.wq : tensor == 1 ? a.wk : a.wv;
  const float* buf = tensor == 0 ? a.bq_in : tensor == 1 ? a.bk_in : a.bv_in;
  void* y = tensor == 0 ? a.q : tensor == 1 ? a.k : a.v;
  const int HD = a.H * D;                          // channels of the tensor
  float s[PL];
  float ss = 0.f;
#pragma unroll
  for (int p = 0; p < PL; ++p) {
    const int c = h * D + PL * lane + p;            // channel in [0, H*D)
    float acc = 0.f;
    for (int i = 0; i < a.K; ++i) {
      const int ti = t - i;
      float xv = 0.f;
      if (ti >= 0) xv = pl_ld<DI>(x, (static_cast<int64_t>(b) * a.T + ti) * HD + c);
      else if (buf != nullptr) xv = buf[(static_cast<int64_t>(b) * (a.K - 1) + (a.K - 1 + ti)) * HD + c];
      acc = fmaf(w[static_cast<int64_t>(i) * HD + c], xv, acc);
    }
    const float sw = acc * sigmoid_f32(acc);
    s[p] = sw;
    ss = fmaf(sw, sw, ss);
  }
  float scale = 1.f;
  if (tensor < 2) scale = 1.f / (sqrtf(wave_sum(ss)) + 1e-12f);
#pragma unroll
  for (int p = 0; p < PL; ++p) pl_st<DO>(y, rr * D + PL * lane + p, s[p] * scale);
}

// new conv buffers: the last K-1 inputs of (old buffer ++ x), one thread per
// (tensor, b, channel); every old value a thread needs is read before it writes.
template <int DI, int D>
__global__ __launch_bounds__(256) void kda_prologue_buf_kernel(PrologueArgs a) {
  const int HD = a.H * D;
  const int64_t n = 3LL * a.B * HD;
  const int64_t id = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (id >= n) return;
  const int tensor = static_cast<int>(id / (static_cast<int64_t>(a.B) * HD));
  const int64_t rem = id - tensor * static_cast<int64_t>(a.B) * HD;
  const int b = static_cast<int>(rem / HD), c = static_cast<int>(rem - static_cast<int64_t>(b) * HD);
  const void* x = tensor == 0 ? a.qp : tensor == 1 ? a.kp : a.vp;
  const float* bin = tensor == 0 ? a.bq_in : tensor == 1 ? a.bk_in : a.bv_in;
  float* bout = tensor == 0 ? a.bq_out : tensor == 1 ? a.bk_out : a.bv_out;
  if (bout == nullptr) return;
  constexpr int KMAX = 8;
  float v[KMAX - 1];
  const int km1 = a.K - 1;
  for (int j = 0; j < km1; ++j) {
    const int src = a.T - km1 + j;                 // row of (old ++ x) relative to x
    float val = 0.f;
    if (src >= 0) val = pl_ld<DI>(x, (static_cast<int64_t>(b) * a.T + src) * HD + c);
    else if (bin != nullptr) val = bin[(static_cast<int64_t>(b) * km1 + (km1 + src)) * HD + c];
    v[j] = val;
  }
  for (int j = 0; j < km1; ++j) bout[(static_cast<int64_t>(b) * km1 + j) * HD + c] = v[j];
}

template <int DO_, int DG, int DY, int D>
__global__ __launch_bounds__(64 * kRowsPerBlock) void kda_epilogue_kernel(EpilogueArgs a) {
  constexpr int PL = D / 64;
  const int lane = threadIdx.x & 63;
  const int64_t rows = static_cast<int64_t>(a.B) * a.T * a.H;
  const int64_t r = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
  if (r >= rows) return;
  float ov[PL];
  float ss = 0.f;
#pragma unroll
  for (int p = 0; p < PL; ++p) {
    ov[p] = pl_ld<DO_>(a.o, r * D + lane + 64 * p);
    ss = fmaf(ov[p], ov[p], ss);
  }
  const float inv = 1.f / sqrtf(wave_sum(ss) / D + a.eps);
#pragma unroll
  for (int p = 0; p < PL; ++p) {
    const float gt = sigmoid_f32(pl_ld<DG>(a.gate, r * D + lane + 64 * p));
    pl_st<DY>(a.y, r * D + lane + 64 * p, gt * ov[p] * inv);
  }
}

template <int D>
hipError_t launch_prologue_d(const PrologueArgs& a, int in_dt, int out_dt, hipStream_t s) {
  const int64_t rows = 3LL * a.B * a.T * a.H;
  const int grid = static_cast<int>((rows + kRowsPerBlock - 1) / kRowsPerBlock);
  if (rows > 0) {
    if (in_dt == 0 && out_dt == 0) hipLaunchKernelGGL((kda_prologue_kernel<0, 0, D>), dim3(grid), dim3(64 * kRowsPerBlock), 0, s, a);
    else if (in_dt == 0) hipLaunchKernelGGL((kda_prologue_kernel<0, 1, D>), dim3(grid), dim3(64 * kRowsPerBlock), 0, s, a);
    else if (out_dt == 0) hipLaunchKernelGGL((kda_prologue_kernel<1, 0, D>), dim3(grid), dim3(64 * kRowsPerBlock), 0, s, a);
    else hipLaunchKernelGGL((kda_prologue_kernel<1, 1, D>), dim3(grid), dim3(64 * kRowsPerBlock), 0, s, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if ((a.bq_out || a.bk_out || a.bv_out) && a.K > 1) {
    const int64_t n = 3LL * a.B * a.H * D;
    const int g = static_cast<int>((n + 255) / 256);
    if (in_dt == 0) hipLaunchKernelGGL((kda_prologue_buf_kernel<0, D>), dim3(g), dim3(256), 0, s, a);
    else hipLaunchKernelGGL((kda_prologue_buf_kernel<1, D>), dim3(g), dim3(256), 0, s, a);
    return hipGetLastError();
  }
  return hipSuccess;
}

template <int D>
hipError_t launch_prologue_buffers_d(const PrologueArgs& a, int in_dt, hipStream_t s) {
  if (!(a.bq_out || a.bk_out || a.bv_out) || a.K <= 1) return hipSuccess;
  const int64_t n = 3LL * a.B * a.H * D;
  const int g = static_cast<int>((n + 255) / 256);
  if (in_dt == 0) hipLaunchKernelGGL((kda_prologue_buf_kernel<0, D>), dim3(g), dim3(256), 0, s, a);
  else hipLaunchKernelGGL((kda_prologue_buf_kernel<1, D>), dim3(g), dim3(256), 0, s, a);
  return hipGetLastError();
}

template <int D>
hipError_t launch_epilogue_d(const EpilogueArgs& a, int o_dt, int g_dt, int y_dt, hipStream_t s) {
  const int64_t rows = static_cast<int64_t>(a.B) * a.T * a.H;
  if (rows == 0) return hipSuccess;
  const int grid = static_cast<int>((rows + kRowsPerBlock - 1) / kRowsPerBlock);
  const int code = o_dt * 4 + g_dt * 2 + y_dt;
  switch (code) {
    case 0: hipLaunchKernelGGL((kda_epilogue_kernel<0, 0, 0, D>), dim3(grid), dim3(64 * kRowsPerBlock), 0, s, a); break;
    case 1: hipLaunchKernelGGL((kda_epilogue_kernel<0, 0, 1, D>), dim3(grid), dim3(64 * kRowsPerBlock), 0, s, a); break;
    case 2: hipLaunchKernelGGL((kda_epilogue_kernel<0, 1, 0, D>), dim3(grid), dim3(64 * kRowsPerBlock), 0, s, a); break;
    case 3: hipLaunchKernelGGL((kda_epilogue_kernel<0, 1, 1, D>), dim3(grid), dim3(64 * kRowsPerBlock), 0, s, a); break;
    case 4: hipLaunchKernelGGL((kda_epilogue_kernel<1, 0, 0, D>), dim3(grid), dim3(64 * kRowsPerBlock), 0, s, a); break;
    case 5: hipLaunchKernelGGL((kda_epilogue_kernel<1, 0, 1, D>), dim3(grid), dim3(64 * kRowsPerBlock), 0, s, a); break;
    case 6: hipLaunchKernelGGL((kda_epilogue_kernel<1, 1, 0, D>), dim3(grid), dim3(64 * kRowsPerBlock), 0, s, a); break;
    default: hipLaunchKernelGGL((kda_epilogue_kernel<1, 1, 1, D>), dim3(grid), dim3(64 * kRowsPerBlock), 0, s, a); break;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_prologue(const PrologueArgs& a, int d, int in_dt, int out_dt, hipStream_t s) {
  return d == 128 ? launch_prologue_d<128>(a, in_dt, out_dt, s) : launch_prologue_d<64>(a, in_dt, out_dt, s);
}

hipError_t launch_prologue_buffers(const PrologueArgs& a, int d, int in_dt, hipStream_t s) {
  return d == 128 ? launch_prologue_buffers_d<128>(a, in_dt, s) : launch_prologue_buffers_d<64>(a, in_dt, s);
}

hipError_t launch_epilogue(const EpilogueArgs& a, int d, int o_dt, int g_dt, int y_dt, hipStream_t s) {
  return d == 128 ? launch_epilogue_d<128>(a, o_dt, g_dt, y_dt, s) : launch_epilogue_d<64>(a, o_dt, g_dt, y_dt, s);
}

}  // namespace kda
