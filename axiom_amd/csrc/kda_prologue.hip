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

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off, 64);
  return x;
}

constexpr int kProRows = 16;   // rows of one (tensor, b, h) per wavefront (T >= 16)

// PL channels of one input row (the bf16 form non-temporal, like the bf16 q,
// k, v stores below: the rows are read by this launch only)
template <int DI, int PL>
__device__ __forceinline__ void pl_ld_pl(const void* p, int64_t i, float (&o)[PL]) {
  if constexpr (DI == 0) {
    if constexpr (PL == 2) {
      const float2 v = *reinterpret_cast<const float2*>(static_cast<const float*>(p) + i);
      o[0] = v.x;
      o[1] = v.y;
    } else {
      o[0] = static_cast<const float*>(p)[i];
    }
  } else {
    if constexpr (PL == 2) {
      const unsigned w = __builtin_nontemporal_load(reinterpret_cast<const unsigned*>(static_cast<const u16*>(p) + i));
      o[0] = __uint_as_float(w << 16);
      o[1] = __uint_as_float(w & 0xFFFF0000u);
    } else {
      o[0] = bf16_to_f32(static_cast<const u16*>(p)[i]);
    }
  }
}

// One wavefront per RW consecutive rows of one (tensor, b, h): the rows and
// the KW-1 before them are loaded once (RW + KW - 1 row loads, all in flight
// together), the K taps run over them in registers, and the row norms are one
// wave_rowsums16 (RW = 16) or one xor-butterfly (RW = 1; the same sums bit for
// bit).  Lane l holds channels PL*l .. PL*l + PL-1 of the head.  BUF (T == 1,
// one wavefront per (tensor, b, h)): the wavefront also writes the new conv
// buffer of its channels -- the old rows 1..K-2 and x -- after reading the old
// one, so in-place buffers need no second launch.
template <int DI, int DO, int D, int KW, int RW, bool BUF>
__global__ __launch_bounds__(64 * kRowsPerBlock) void kda_prologue_kernel(PrologueArgs a) {
  constexpr int kProRows = RW;
  constexpr int PL = D / 64;   // channels per lane
  const int lane = threadIdx.x & 63;
  const int nblk = (a.T + kProRows - 1) / kProRows;
  const int64_t items = 3LL * a.B * a.H * nblk;
  const int64_t w = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + (threadIdx.x >> 6);
  if (w >= items) return;                          // uniform per wavefront
  const int blk = static_cast<int>(w % nblk);
  int64_t rest = w / nblk;
  const int h = static_cast<int>(rest % a.H);
  rest /= a.H;
  const int b = static_cast<int>(rest % a.B);
  const int tensor = static_cast<int>(rest / a.B);  // 0 q, 1 k, 2 v
  const void* x = tensor == 0 ? a.qp : tensor == 1 ? a.kp : a.vp;
  const float* wp = tensor == 0 ? a.wq : tensor == 1 ? a.wk : a.wv;
  const float* buf = tensor == 0 ? a.bq_in : tensor == 1 ? a.bk_in : a.bv_in;
  void* y = tensor == 0 ? a.q : tensor == 1 ? a.k : a.v;
  const int HD = a.H * D;
  const int c0 = h * D + PL * lane;                // the lane's first channel in [0, H*D)
  const int t0 = blk * kProRows;
  float wt[KW][PL];
#pragma unroll
  for (int i = 0; i < KW; ++i) {
    const float* p = wp + static_cast<int64_t>(min(i, a.K - 1)) * HD + c0;
#pragma unroll
    for (int q = 0; q < PL; ++q) wt[i][q] = p[q];
  }
  // xs[j] = input row t0 - (KW-1) + j; rows before the sequence from the
  // buffer (or zero), rows past its end re-read the last row (never stored)
  float xs[KW - 1 + kProRows][PL];
#pragma unroll
  for (int j = 0; j < KW - 1; ++j) {
    const int tr = t0 - (KW - 1) + j;                // uniform per wavefront
    if (tr >= 0) {
      pl_ld_pl<DI, PL>(x, (static_cast<int64_t>(b) * a.T + tr) * HD + c0, xs[j]);
    } else {
      const int br = a.K - 1 + tr;                   // buffer row (oldest first)
#pragma unroll
      for (int q = 0; q < PL; ++q)
        xs[j][q] = (buf != nullptr && br >= 0) ? buf[(static_cast<int64_t>(b) * (a.K - 1) + br) * HD + c0 + q] : 0.f;
    }
  }
#pragma unroll
  for (int r = 0; r < kProRows; ++r)
    pl_ld_pl<DI, PL>(x, (static_cast<int64_t>(b) * a.T + min(t0 + r, a.T - 1)) * HD + c0, xs[KW - 1 + r]);
  float sv[kProRows][PL], ss[kProRows];
#pragma unroll
  for (int r = 0; r < kProRows; ++r) {
    ss[r] = 0.f;
#pragma unroll
    for (int q = 0; q < PL; ++q) {
      float acc = 0.f;
#pragma unroll
      for (int i = 0; i < KW; ++i)
        if (i < a.K) acc = fmaf(wt[i][q], xs[KW - 1 + r - i][q], acc);
      sv[r][q] = acc * sigmoid_f32(acc);
      ss[r] = fmaf(sv[r][q], sv[r][q], ss[r]);
    }
  }
  if (tensor < 2) {
    float tot[kProRows];
    if constexpr (RW == 16) wave_rowsums16(ss, tot);
    else tot[0] = wave_sum(ss[0]);
#pragma unroll
    for (int r = 0; r < kProRows; ++r) {
      const float sc = inv_l2_f32(tot[r]);
#pragma unroll
      for (int q = 0; q < PL; ++q) sv[r][q] *= sc;
    }
  }
  if constexpr (BUF) {
    // new buffer row j = (old ++ x)[1 + j] = xs[KW - K + 1 + j]
    float* bout = tensor == 0 ? a.bq_out : tensor == 1 ? a.bk_out : a.bv_out;
    if (bout != nullptr) {
#pragma unroll
      for (int j = 0; j < KW - 1; ++j) {
        if (j >= a.K - 1) break;
#pragma unroll
        for (int q = 0; q < PL; ++q)
          bout[(static_cast<int64_t>(b) * (a.K - 1) + j) * HD + c0 + q] = xs[KW - a.K + 1 + j][q];
      }
    }
  }
#pragma unroll
  for (int r = 0; r < kProRows; ++r) {
    if (t0 + r >= a.T) break;
    const int64_t o = ((static_cast<int64_t>(b) * a.T + t0 + r) * a.H + h) * D + PL * lane;
    if constexpr (DO == 0) {
      if constexpr (PL == 2) *reinterpret_cast<float2*>(static_cast<float*>(y) + o) = make_float2(sv[r][0], sv[r][1]);
      else static_cast<float*>(y)[o] = sv[r][0];
    } else {
      if constexpr (PL == 2) __builtin_nontemporal_store(pack_bf16x2(sv[r][0], sv[r][1]), reinterpret_cast<unsigned*>(static_cast<u16*>(y) + o));
      else static_cast<u16*>(y)[o] = cvt_bf16(sv[r][0]);
    }
  }
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

// Four consecutive channels per lane: a row of D channels is D/4 lanes (a
// half wavefront at D = 128), the head's sum of squares a butterfly inside
// that lane group; 16-byte o loads, 8-byte bf16 gate loads and y stores, all
// non-temporal (each element is touched once: epilogue 89 -> 74 us backward,
// layer 324 -> 314 us, when introduced).
// kEpiRowsPerBlock rows per workgroup per step, grid-strided.
constexpr int kEpiThreads = 256;

template <int DT>
__device__ __forceinline__ f4 ep_ld4(const void* p, int64_t i) {
  if constexpr (DT == 0) {
    return __builtin_nontemporal_load(reinterpret_cast<const f4*>(static_cast<const float*>(p) + i));
  } else {
    typedef unsigned int u2v __attribute__((ext_vector_type(2)));
    const u2v w = __builtin_nontemporal_load(reinterpret_cast<const u2v*>(static_cast<const u16*>(p) + i));
    return f4{__uint_as_float(w.x << 16), __uint_as_float(w.x & 0xFFFF0000u), __uint_as_float(w.y << 16),
              __uint_as_float(w.y & 0xFFFF0000u)};
  }
}

template <int DT>
__device__ __forceinline__ void ep_st4(void* p, int64_t i, const f4& v) {
  if constexpr (DT == 0) {
    __builtin_nontemporal_store(v, reinterpret_cast<f4*>(static_cast<float*>(p) + i));
  } else {
    typedef unsigned int u2v __attribute__((ext_vector_type(2)));
    __builtin_nontemporal_store(u2v{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])}, reinterpret_cast<u2v*>(static_cast<u16*>(p) + i));
  }
}

template <int DO_, int DG, int DY, int D>
__global__ __launch_bounds__(kEpiThreads) void kda_epilogue_kernel(EpilogueArgs a) {
  constexpr int LPR = D / 4;                    // lanes per row
  constexpr int RPB = kEpiThreads / LPR;        // rows per workgroup step
  const int64_t rows = static_cast<int64_t>(a.B) * a.T * a.H;
  const int sub = threadIdx.x % LPR;
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * RPB + threadIdx.x / LPR; r < rows;
       r += static_cast<int64_t>(gridDim.x) * RPB) {   // a row's lanes share r: uniform per group
    const int64_t i = r * D + 4 * sub;
    const f4 o = ep_ld4<DO_>(a.o, i);
    const f4 g = ep_ld4<DG>(a.gate, i);
    float ss = o[0] * o[0];
#pragma unroll
    for (int e = 1; e < 4; ++e) ss = fmaf(o[e], o[e], ss);
#pragma unroll
    for (int off = LPR / 2; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, 64);
    const float inv = __builtin_amdgcn_rsqf(ss * (1.f / D) + a.eps);
    f4 y;
#pragma unroll
    for (int e = 0; e < 4; ++e) y[e] = sigmoid_f32(g[e]) * o[e] * inv;
    ep_st4<DY>(a.y, i, y);
  }
}

template <int D, int KW, int RW, bool BUF>
void launch_prologue_main(const PrologueArgs& a, int in_dt, int out_dt, int grid, hipStream_t s) {
  const dim3 g(grid), blk(64 * kRowsPerBlock);
  if (in_dt == 0 && out_dt == 0) hipLaunchKernelGGL((kda_prologue_kernel<0, 0, D, KW, RW, BUF>), g, blk, 0, s, a);
  else if (in_dt == 0) hipLaunchKernelGGL((kda_prologue_kernel<0, 1, D, KW, RW, BUF>), g, blk, 0, s, a);
  else if (out_dt == 0) hipLaunchKernelGGL((kda_prologue_kernel<1, 0, D, KW, RW, BUF>), g, blk, 0, s, a);
  else hipLaunchKernelGGL((kda_prologue_kernel<1, 1, D, KW, RW, BUF>), g, blk, 0, s, a);
}

template <int D, int RW, bool BUF>
void launch_prologue_k(const PrologueArgs& a, int in_dt, int out_dt, hipStream_t s) {
  const int64_t items = 3LL * a.B * a.H * ((a.T + RW - 1) / RW);
  const int grid = static_cast<int>((items + kRowsPerBlock - 1) / kRowsPerBlock);
  if (a.K <= 4) launch_prologue_main<D, 4, RW, BUF>(a, in_dt, out_dt, grid, s);
  else launch_prologue_main<D, 8, RW, BUF>(a, in_dt, out_dt, grid, s);
}

template <int D>
hipError_t launch_prologue_d(const PrologueArgs& a, int in_dt, int out_dt, hipStream_t s) {
  // T == 1 (a decode step): one wavefront per (tensor, b, h), buffers written
  // by the same kernel; short sequences one row per wavefront; else 16.
  if (a.T == 1) {
    launch_prologue_k<D, 1, true>(a, in_dt, out_dt, s);
    return hipGetLastError();
  }
  if (a.T > 0) {
    if (a.T < kProRows) launch_prologue_k<D, 1, false>(a, in_dt, out_dt, s);
    else launch_prologue_k<D, kProRows, false>(a, in_dt, out_dt, s);
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
  constexpr int RPB = kEpiThreads / (D / 4);
  const int64_t need = (rows + RPB - 1) / RPB;
  const int grid = static_cast<int>(need < 8192 ? need : 8192);   // 32 workgroups per CU, grid-strided
  const int code = o_dt * 4 + g_dt * 2 + y_dt;
  switch (code) {
    case 0: hipLaunchKernelGGL((kda_epilogue_kernel<0, 0, 0, D>), dim3(grid), dim3(kEpiThreads), 0, s, a); break;
    case 1: hipLaunchKernelGGL((kda_epilogue_kernel<0, 0, 1, D>), dim3(grid), dim3(kEpiThreads), 0, s, a); break;
    case 2: hipLaunchKernelGGL((kda_epilogue_kernel<0, 1, 0, D>), dim3(grid), dim3(kEpiThreads), 0, s, a); break;
    case 3: hipLaunchKernelGGL((kda_epilogue_kernel<0, 1, 1, D>), dim3(grid), dim3(kEpiThreads), 0, s, a); break;
    case 4: hipLaunchKernelGGL((kda_epilogue_kernel<1, 0, 0, D>), dim3(grid), dim3(kEpiThreads), 0, s, a); break;
    case 5: hipLaunchKernelGGL((kda_epilogue_kernel<1, 0, 1, D>), dim3(grid), dim3(kEpiThreads), 0, s, a); break;
    case 6: hipLaunchKernelGGL((kda_epilogue_kernel<1, 1, 0, D>), dim3(grid), dim3(kEpiThreads), 0, s, a); break;
    default: hipLaunchKernelGGL((kda_epilogue_kernel<1, 1, 1, D>), dim3(grid), dim3(kEpiThreads), 0, s, a); break;
  }
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Backward of the prologue.  With a = conv(x), sg = sigmoid(a), s = a sg and,
// for q and k, y = s / (||s|| + 1e-12) (y = s for v):
//   ds = dy / (n + eps) - s (s . dy) / (n (n + eps)^2), n = ||s|| (0 when n = 0:
//        the reference's tangent convention at a zero row), or ds = dy for v;
//   da = ds sg (1 + a (1 - sg));
//   dx[t] = sum_i w[i] da[t + i];  dbuf[j] = the same sum at the history row
//   j - (K-1);  dw[i] = sum_t da[t] x[t - i].
// One pass: a wavefront owns 16 rows of one (tensor, b, h) and recomputes the
// forward, and da, for those rows and the K-1 rows after them (the halo its dx
// sums reach), so da never goes through memory.  A workgroup is four
// wavefronts on 64 consecutive rows; it adds its dw sums in LDS and writes one
// partial sum per 64-row group, which a second launch reduces.
// ---------------------------------------------------------------------------
// arr[t] for a wave-uniform t < 3 by scalar selects (a runtime index into
// the kernel-argument struct would read it through memory)
template <typename P>
__device__ __forceinline__ P pick3(const P (&arr)[3], int t) {
  return t == 0 ? arr[0] : (t == 1 ? arr[1] : arr[2]);
}

// PL consecutive channels at element offset lo of a row whose address is
// wave-uniform (scalar base + 32-bit lane offset).
template <int DI, int PL>
__device__ __forceinline__ void ld_row(const void* row, unsigned lo, float (&o)[PL]) {
  if constexpr (DI == 0) {
    const float* p = static_cast<const float*>(row) + lo;
    if constexpr (PL == 2) {
      const float2 v = *reinterpret_cast<const float2*>(p);
      o[0] = v.x;
      o[1] = v.y;
    } else {
      o[0] = p[0];
    }
  } else {
    const u16* p = static_cast<const u16*>(row) + lo;
    if constexpr (PL == 2) {
      const unsigned w = *reinterpret_cast<const unsigned*>(p);
      o[0] = __uint_as_float(w << 16);
      o[1] = __uint_as_float(w & 0xFFFF0000u);
    } else {
      o[0] = bf16_to_f32(p[0]);
    }
  }
}

template <int DI, int D, int KW>
__global__ __launch_bounds__(64 * kRowsPerBlock) void kda_prologue_bwd_kernel(PrologueBwdArgs a) {
  constexpr int RW = 16;
  constexpr int HW = KW - 1;      // halo rows (da after the block; x before it)
  constexpr int PL = D / 64;
  constexpr int ES = DI == 0 ? 4 : 2;
  __shared__ float sPart[kRowsPerBlock][KW][64 * PL];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = blockIdx.x % a.G;                  // 64-row group
  int rest = blockIdx.x / a.G;
  const int h = rest % a.H;
  rest /= a.H;
  const int b = rest % a.B;
  const int tensor = rest / a.B;
  const int HD = a.H * D;
  const unsigned lo = PL * lane;
  const int t0 = 64 * g + RW * wv;
  // wave-uniform bases at (b, row 0, channel h * D)
  const int64_t rowbase = static_cast<int64_t>(b) * a.T * HD + h * D;
  const char* xb = static_cast<const char*>(pick3(a.x, tensor)) + rowbase * ES;
  const float* yb = pick3(a.dy, tensor) + rowbase;
  const float* buf = pick3(a.bin, tensor);
  const float* bb = buf == nullptr ? nullptr : buf + static_cast<int64_t>(b) * (a.K - 1) * HD + h * D;
  float wt[KW][PL];                // taps K .. KW-1 are zero: every sum below runs over KW
#pragma unroll
  for (int i = 0; i < KW; ++i) {
    float w[PL];
    ld_row<0, PL>(pick3(a.w, tensor) + static_cast<int64_t>(min(i, a.K - 1)) * HD + h * D, lo, w);
#pragma unroll
    for (int q = 0; q < PL; ++q) wt[i][q] = i < a.K ? w[q] : 0.f;
  }
  // x rows t0 - HW .. t0 + RW + HW - 1 and dy rows t0 .. t0 + RW + HW - 1,
  // loaded from clamped rows without branches (every load in flight at once);
  // the few edge rows are fixed up after: before row 0 the carried buffer or
  // zeros, dy zero from T on (so da is zero there)
  float xs[RW + 2 * HW][PL];
  float dd[RW + HW][PL];
#pragma unroll
  for (int j = 0; j < RW + 2 * HW; ++j)
    ld_row<DI, PL>(xb + static_cast<int64_t>(min(max(t0 - HW + j, 0), a.T - 1)) * HD * ES, lo, xs[j]);
#pragma unroll
  for (int r = 0; r < RW + HW; ++r) ld_row<0, PL>(yb + static_cast<int64_t>(min(t0 + r, a.T - 1)) * HD, lo, dd[r]);
  if (t0 == 0) {
#pragma unroll
    for (int j = 0; j < HW; ++j) {
      const int br = a.K - 1 - HW + j;      // buffer row of sequence row j - HW
      if (bb != nullptr && br >= 0) {
        ld_row<0, PL>(bb + static_cast<int64_t>(br) * HD, lo, xs[j]);
      } else {
#pragma unroll
        for (int q = 0; q < PL; ++q) xs[j][q] = 0.f;
      }
    }
  }
  if (t0 + RW + HW > a.T) {
#pragma unroll
    for (int r = 0; r < RW + HW; ++r)
      if (t0 + r >= a.T) {
#pragma unroll
        for (int q = 0; q < PL; ++q) dd[r][q] = 0.f;
      }
  }
  // s = a sg and the swish derivative f = sg (1 + a (1 - sg)) per element
  float sv[RW + HW][PL], fv[RW + HW][PL];
#pragma unroll
  for (int r = 0; r < RW + HW; ++r)
#pragma unroll
    for (int q = 0; q < PL; ++q) {
      float av = 0.f;
#pragma unroll
      for (int i = 0; i < KW; ++i) av = fmaf(wt[i][q], xs[HW + r - i][q], av);
      const float sg = sigmoid_f32(av);
      sv[r][q] = av * sg;
      fv[r][q] = sg * fmaf(av, 1.f - sg, 1.f);
    }
  if (tensor < 2) {
    float c1[RW], c2[RW], h1[HW], h2[HW];
#pragma unroll
    for (int r = 0; r < RW + HW; ++r) {
      float ss = 0.f, sd = 0.f;
#pragma unroll
      for (int q = 0; q < PL; ++q) {
        ss = fmaf(sv[r][q], sv[r][q], ss);
        sd = fmaf(sv[r][q], dd[r][q], sd);
      }
      if (r < RW) {
        c1[r] = ss;
        c2[r] = sd;
      } else {
        h1[r - RW] = wave_sum(ss);
        h2[r - RW] = wave_sum(sd);
      }
    }
    // ds = dy k1 - s k2 with k1 = 1 / (n + eps), k2 = (s . dy) / (n (n + eps)^2)
    // (both 0 when n = 0), evaluated once per lane for the 16 rows it holds
    auto coef = [](float nsq, float sdr, float& k1, float& k2) {
      const float n = __builtin_amdgcn_sqrtf(nsq);
      const float npe = n + 1e-12f;
      k1 = n > 0.f ? __builtin_amdgcn_rcpf(npe) : 0.f;
      k2 = n > 0.f ? sdr * __builtin_amdgcn_rcpf(n * npe * npe) : 0.f;
    };
    float k1v, k2v;
    coef(wave_rowsums16_lanes(c1), wave_rowsums16_lanes(c2), k1v, k2v);
#pragma unroll
    for (int r = 0; r < RW + HW; ++r) {
      float k1, k2;
      if (r < RW) {
        k1 = readlane_f32(k1v, rowsum16_lane(r));
        k2 = readlane_f32(k2v, rowsum16_lane(r));
      } else {
        coef(h1[r - RW], h2[r - RW], k1, k2);
      }
#pragma unroll
      for (int q = 0; q < PL; ++q) dd[r][q] = fmaf(dd[r][q], k1, -sv[r][q] * k2) * fv[r][q];
    }
  } else {
#pragma unroll
    for (int r = 0; r < RW + HW; ++r)
#pragma unroll
      for (int q = 0; q < PL; ++q) dd[r][q] *= fv[r][q];
  }
  // dx
  float* xo = pick3(a.dx, tensor) + rowbase;
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    if (t0 + r >= a.T) break;
    float acc[PL];
#pragma unroll
    for (int q = 0; q < PL; ++q) {
      acc[q] = 0.f;
#pragma unroll
      for (int i = 0; i < KW; ++i) acc[q] = fmaf(wt[i][q], dd[r + i][q], acc[q]);
    }
    float* p = xo + static_cast<int64_t>(t0 + r) * HD + lo;
    if constexpr (PL == 2) *reinterpret_cast<float2*>(p) = make_float2(acc[0], acc[1]);
    else p[0] = acc[0];
  }
  // the incoming buffer: sequence row -m (m = 1 .. K-1) is its row K-1-m and
  // reaches the outputs 0 .. KW-1-m through taps m .. KW-1
  float* dbp = pick3(a.db, tensor);
  if (t0 == 0 && dbp != nullptr) {
    float* dbb = dbp + static_cast<int64_t>(b) * (a.K - 1) * HD + h * D + lo;
#pragma unroll
    for (int m = 1; m <= HW; ++m) {
      if (m > a.K - 1) break;
#pragma unroll
      for (int q = 0; q < PL; ++q) {
        float acc = 0.f;
#pragma unroll
        for (int i = m; i < KW; ++i) acc = fmaf(wt[i][q], dd[i - m][q], acc);
        dbb[static_cast<int64_t>(a.K - 1 - m) * HD + q] = acc;
      }
    }
  }
  // dw sums over this wavefront's rows (da = 0 from T on), then over the four
#pragma unroll
  for (int i = 0; i < KW; ++i)
#pragma unroll
    for (int q = 0; q < PL; ++q) {
      float acc = 0.f;
#pragma unroll
      for (int r = 0; r < RW; ++r) acc = fmaf(dd[r][q], xs[HW + r - i][q], acc);
      sPart[wv][i][lo + q] = acc;
    }
  __syncthreads();
  if (wv == 0) {
    float* pp = a.part + (static_cast<int64_t>(tensor) * a.B * a.G + static_cast<int64_t>(b) * a.G + g) * a.K * HD +
                h * D;
#pragma unroll
    for (int i = 0; i < KW; ++i) {
      if (i >= a.K) break;
#pragma unroll
      for (int q = 0; q < PL; ++q) {
        const int c = lo + q;
        pp[static_cast<int64_t>(i) * HD + c] = ((sPart[0][i][c] + sPart[1][i][c]) + sPart[2][i][c]) + sPart[3][i][c];
      }
    }
  }
}

// dw[tensor][i][c] = sum of the B * G partial sums.  A workgroup takes 64
// columns of one (tensor, i); its eight wavefronts take every eighth partial
// (four loads in flight each), then add in LDS.  With T == 0 the blocks after
// those zero the buffers' gradients (no output reads the buffers).
constexpr int kDwWaves = 8;

__global__ __launch_bounds__(64 * kDwWaves) void kda_prologue_bwd_dw_kernel(PrologueBwdArgs a, int HD) {
  __shared__ float sSum[kDwWaves][64];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int cb = HD / 64;
  const int ndw = 3 * a.K * cb;
  if (static_cast<int>(blockIdx.x) < ndw) {
    const int tensor = blockIdx.x / (a.K * cb);
    const int rem = blockIdx.x % (a.K * cb);
    const int i = rem / cb;
    const int c = (rem % cb) * 64 + lane;
    const int64_t stride = static_cast<int64_t>(a.K) * HD;
    const float* pp = a.part + static_cast<int64_t>(tensor) * a.B * a.G * stride + static_cast<int64_t>(i) * HD + c;
    const int np = a.B * a.G;
    float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
    int p = wv;
    for (; p + 3 * kDwWaves < np; p += 4 * kDwWaves) {
      s0 += pp[p * stride];
      s1 += pp[(p + kDwWaves) * stride];
      s2 += pp[(p + 2 * kDwWaves) * stride];
      s3 += pp[(p + 3 * kDwWaves) * stride];
    }
    for (; p < np; p += kDwWaves) s0 += pp[p * stride];
    sSum[wv][lane] = (s0 + s1) + (s2 + s3);
    __syncthreads();
    if (wv == 0) {
      float acc = 0.f;
#pragma unroll
      for (int w = 0; w < kDwWaves; ++w) acc += sSum[w][lane];
      pick3(a.dw, tensor)[static_cast<int64_t>(i) * HD + c] = acc;
    }
  } else if (a.T == 0) {
    const int64_t per = static_cast<int64_t>(a.B) * (a.K - 1) * HD;
    const int64_t j = static_cast<int64_t>(blockIdx.x - ndw) * (64 * kDwWaves) + threadIdx.x;
    if (j < 3 * per) {
      const int tensor = static_cast<int>(j / per);
      float* dbp = pick3(a.db, tensor);
      if (dbp != nullptr) dbp[j - tensor * per] = 0.f;
    }
  }
}

template <int D, int KW>
hipError_t launch_prologue_bwd_k(const PrologueBwdArgs& a, int in_dt, hipStream_t s) {
  if (a.T > 0) {
    const int grid = 3 * a.B * a.H * a.G;
    if (in_dt == 0) hipLaunchKernelGGL((kda_prologue_bwd_kernel<0, D, KW>), dim3(grid), dim3(64 * kRowsPerBlock), 0, s, a);
    else hipLaunchKernelGGL((kda_prologue_bwd_kernel<1, D, KW>), dim3(grid), dim3(64 * kRowsPerBlock), 0, s, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  const int HD = a.H * D;
  int64_t blocks = 3LL * a.K * (HD / 64);
  if (a.T == 0) blocks += (3LL * a.B * (a.K - 1) * HD + 64 * kDwWaves - 1) / (64 * kDwWaves);
  hipLaunchKernelGGL(kda_prologue_bwd_dw_kernel, dim3(static_cast<int>(blocks)), dim3(64 * kDwWaves), 0, s, a, HD);
  return hipGetLastError();
}

// Epilogue backward: y = sg o r with sg = sigmoid(z), r = (mean(o^2) + eps)^-1/2:
//   dz = dy o r sg (1 - sg);  do = sg r dy - o r^3 (sum_c dy sg o) / D.
// Same layout as the epilogue: four channels per lane, D/4 lanes per row.
template <int DO_, int DG, int DDY, int DDG, int D>
__global__ __launch_bounds__(kEpiThreads) void kda_epilogue_bwd_kernel(EpilogueBwdArgs a) {
  constexpr int LPR = D / 4;
  constexpr int RPB = kEpiThreads / LPR;
  const int64_t rows = static_cast<int64_t>(a.B) * a.T * a.H;
  const int sub = threadIdx.x % LPR;
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * RPB + threadIdx.x / LPR; r < rows;
       r += static_cast<int64_t>(gridDim.x) * RPB) {
    const int64_t i = r * D + 4 * sub;
    const f4 o = ep_ld4<DO_>(a.o, i);
    const f4 z = ep_ld4<DG>(a.gate, i);
    const f4 dy = ep_ld4<DDY>(a.dy, i);
    f4 sg;
    float ss = 0.f, sd = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      sg[e] = sigmoid_f32(z[e]);
      ss = fmaf(o[e], o[e], ss);
      sd = fmaf(dy[e] * sg[e], o[e], sd);
    }
#pragma unroll
    for (int off = LPR / 2; off >= 1; off >>= 1) {
      ss += __shfl_xor(ss, off, 64);
      sd += __shfl_xor(sd, off, 64);
    }
    const float rr = __builtin_amdgcn_rsqf(ss * (1.f / D) + a.eps);
    const float c3 = rr * rr * rr * sd * (1.f / D);
    f4 dz, dout;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      dz[e] = dy[e] * o[e] * rr * sg[e] * (1.f - sg[e]);
      dout[e] = sg[e] * rr * dy[e] - o[e] * c3;
    }
    *reinterpret_cast<float4*>(a.dout + i) = make_float4(dout[0], dout[1], dout[2], dout[3]);
    ep_st4<DDG>(a.dgate, i, dz);
  }
}

template <int D>
hipError_t launch_epilogue_bwd_d(const EpilogueBwdArgs& a, int o_dt, int g_dt, int dy_dt, int dg_dt, hipStream_t s) {
  const int64_t rows = static_cast<int64_t>(a.B) * a.T * a.H;
  if (rows == 0) return hipSuccess;
  constexpr int RPB = kEpiThreads / (D / 4);
  const int64_t need = (rows + RPB - 1) / RPB;
  const dim3 grid(static_cast<int>(need < 8192 ? need : 8192)), blk(kEpiThreads);
  const int code = o_dt * 8 + g_dt * 4 + dy_dt * 2 + dg_dt;
#define KDA_EPB(C, A, B2, Cc, Dd) \
  case C: hipLaunchKernelGGL((kda_epilogue_bwd_kernel<A, B2, Cc, Dd, D>), grid, blk, 0, s, a); break;
  switch (code) {
    KDA_EPB(0, 0, 0, 0, 0) KDA_EPB(1, 0, 0, 0, 1) KDA_EPB(2, 0, 0, 1, 0) KDA_EPB(3, 0, 0, 1, 1)
    KDA_EPB(4, 0, 1, 0, 0) KDA_EPB(5, 0, 1, 0, 1) KDA_EPB(6, 0, 1, 1, 0) KDA_EPB(7, 0, 1, 1, 1)
    KDA_EPB(8, 1, 0, 0, 0) KDA_EPB(9, 1, 0, 0, 1) KDA_EPB(10, 1, 0, 1, 0) KDA_EPB(11, 1, 0, 1, 1)
    KDA_EPB(12, 1, 1, 0, 0) KDA_EPB(13, 1, 1, 0, 1) KDA_EPB(14, 1, 1, 1, 0) default:
      hipLaunchKernelGGL((kda_epilogue_bwd_kernel<1, 1, 1, 1, D>), grid, blk, 0, s, a); break;
  }
#undef KDA_EPB
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

namespace kda {

hipError_t launch_prologue_bwd(const PrologueBwdArgs& a, int d, int in_dt, hipStream_t s) {
  if (d == 128) return a.K <= 4 ? launch_prologue_bwd_k<128, 4>(a, in_dt, s) : launch_prologue_bwd_k<128, 8>(a, in_dt, s);
  return a.K <= 4 ? launch_prologue_bwd_k<64, 4>(a, in_dt, s) : launch_prologue_bwd_k<64, 8>(a, in_dt, s);
}

hipError_t launch_epilogue_bwd(const EpilogueBwdArgs& a, int d, int o_dt, int g_dt, int dy_dt, int dg_dt,
                               hipStream_t s) {
  return d == 128 ? launch_epilogue_bwd_d<128>(a, o_dt, g_dt, dy_dt, dg_dt, s)
                  : launch_epilogue_bwd_d<64>(a, o_dt, g_dt, dy_dt, dg_dt, s);
}

}  // namespace kda
