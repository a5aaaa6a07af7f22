// Standalone batched unit-triangular solve: X = (I + L)^-1 B or
// X = (I + L)^-T B per head, L = strict lower part of a [H][C][C] (C <= 64),
// B [H][C][N] -- the drop-in for the reference's UT-solve kernels
// (net/kernels/kda_ut_solve.py:525 kernel, :536 kernel_t) -- and the backward
// rule of their custom_vjp (:563 _backward): dB = the sibling solve of dX,
// dA = strict_lower(-dB X^T) (or strict_lower(-X dB^T) for the transposed
// solve).  fp32 arithmetic; a, b, x fp32 or bf16.
//
// One workgroup per (head, 64-column tile of B): L (zero-padded to 64 x 64)
// and the B tile go to LDS, T = (I + L)^-1 is formed there (kda_tri.h), and
// X = T B (or T^T B) is an LDS-tiled FMA product, each thread owning 4 x 4
// outputs.  Padding rows/columns beyond C and N are zero and never stored.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "kda_common.h"
#include "kda_internal.h"
#include "kda_tri.h"

namespace kda {
namespace {

constexpr int kN = 64;        // padded size
constexpr int kPC = kN + 1;   // LDS pitch
constexpr int kUtThreads = 256;

template <int DT>
__device__ __forceinline__ float ut_ld(const void* p, int64_t i) {
  if constexpr (DT == 0) return static_cast<const float*>(p)[i];
  else return bf16_to_f32(static_cast<const u16*>(p)[i]);
}

template <int DT>
__device__ __forceinline__ void ut_st(void* p, int64_t i, float v) {
  if constexpr (DT == 0) static_cast<float*>(p)[i] = v;
  else static_cast<u16*>(p)[i] = f32_to_bf16_bits(v);
}

// Forward solve (B = b) or backward rule (B = dX; db written to x, and with
// `da` set, dA from the forward solution `xf`).
template <int DT, bool TR>
__global__ __launch_bounds__(kUtThreads) void kda_ut_solve_kernel(UtArgs a) {
  __shared__ float sL[kN * kPC], sT[kN * kPC], sB[kN * kPC], tmp[768];
  const int t = threadIdx.x, rm = t >> 4, cn = t & 15;
  const int h = blockIdx.x / a.ntiles, tile = blockIdx.x - h * a.ntiles;
  const int j0 = kN * tile;
  const int C = a.C, N = a.N;
  const int64_t abase = static_cast<int64_t>(h) * C * C;
  const int64_t bbase = static_cast<int64_t>(h) * C * N;
  for (int e = t; e < kN * kN; e += kUtThreads) {
    const int c = e >> 6, i = e & 63;
    sL[c * kPC + i] = (c < C && i < c) ? ut_ld<DT>(a.a, abase + static_cast<int64_t>(c) * C + i) : 0.f;
    sB[c * kPC + i] = (c < C && j0 + i < N) ? ut_ld<DT>(a.b, bbase + static_cast<int64_t>(c) * N + j0 + i) : 0.f;
  }
  __syncthreads();
  invert_unit_lower64<kPC, kUtThreads>(sL, sT, tmp);
  float acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.f;
#pragma unroll 4
  for (int m = 0; m < kN; ++m) {
    float tv[4], bv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) tv[i] = TR ? sT[m * kPC + rm + 16 * i] : sT[(rm + 16 * i) * kPC + m];
#pragma unroll
    for (int j = 0; j < 4; ++j) bv[j] = sB[m * kPC + cn + 16 * j];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(tv[i], bv[j], acc[i][j]);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = rm + 16 * i, col = j0 + cn + 16 * j;
      if (c < C && col < N) ut_st<DT>(a.x, bbase + static_cast<int64_t>(c) * N + col, acc[i][j]);
    }
}

// dA[h] = strict_lower(-Y X^T) (TR = false: Y = db, X = forward solution) or
// strict_lower(-X Y^T) (TR = true); one workgroup per head, K = N in tiles of 64.
template <int DT, bool TR>
__global__ __launch_bounds__(kUtThreads) void kda_ut_da_kernel(UtArgs a) {
  __shared__ float sY[kN * kPC], sX[kN * kPC];
  const int t = threadIdx.x, rm = t >> 4, cn = t & 15;
  const int h = blockIdx.x;
  const int C = a.C, N = a.N;
  const int64_t bbase = static_cast<int64_t>(h) * C * N;
  // P = sum_n R[c][n] Q[i][n] with R = Y, Q = X (TR: R = X, Q = Y)
  const void* Rp = TR ? a.xf : a.x;
  const void* Qp = TR ? a.x : a.xf;
  float acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.f;
  for (int n0 = 0; n0 < N; n0 += kN) {
    for (int e = t; e < kN * kN; e += kUtThreads) {
      const int c = e >> 6, n = e & 63;
      const bool in = c < C && n0 + n < N;
      sY[c * kPC + n] = in ? ut_ld<DT>(Rp, bbase + static_cast<int64_t>(c) * N + n0 + n) : 0.f;
      sX[c * kPC + n] = in ? ut_ld<DT>(Qp, bbase + static_cast<int64_t>(c) * N + n0 + n) : 0.f;
    }
    __syncthreads();
#pragma unroll 4
    for (int n = 0; n < kN; ++n) {
      float rv[4], qv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) rv[i] = sY[(rm + 16 * i) * kPC + n];
#pragma unroll
      for (int j = 0; j < 4; ++j) qv[j] = sX[(cn + 16 * j) * kPC + n];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(rv[i], qv[j], acc[i][j]);
    }
    __syncthreads();
  }
  const int64_t abase = static_cast<int64_t>(h) * C * C;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = rm + 16 * i, col = cn + 16 * j;
      if (c < C && col < C) ut_st<DT>(a.da, abase + static_cast<int64_t>(c) * C + col, (col < c) ? -acc[i][j] : 0.f);
    }
}

template <int DT>
hipError_t launch_ut_t(const UtArgs& a, bool transpose, bool with_da, hipStream_t s) {
  const int grid = a.H * a.ntiles;
  if (transpose) hipLaunchKernelGGL((kda_ut_solve_kernel<DT, true>), dim3(grid), dim3(kUtThreads), 0, s, a);
  else hipLaunchKernelGGL((kda_ut_solve_kernel<DT, false>), dim3(grid), dim3(kUtThreads), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || !with_da) return e;
  // the backward of the forward solve runs the transposed solve, and vice
  // versa; `transpose` here is the solve just run, so the dA form is its
  // opposite: forward solve's backward (transpose == true) uses -Y X^T
  if (transpose) hipLaunchKernelGGL((kda_ut_da_kernel<DT, false>), dim3(a.H), dim3(kUtThreads), 0, s, a);
  else hipLaunchKernelGGL((kda_ut_da_kernel<DT, true>), dim3(a.H), dim3(kUtThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_ut(const UtArgs& a, int dtype, bool transpose, bool with_da, hipStream_t s) {
  return dtype == 0 ? launch_ut_t<0>(a, transpose, with_da, s) : launch_ut_t<1>(a, transpose, with_da, s);
}

}  // namespace kda
