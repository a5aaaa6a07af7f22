// Standalone batched unit-triangular solve: X = (I + L)^-1 B or
// X = (I + L)^-T B per head, L = strict lower part of a [H][C][C] (C <= 64),
// B [H][C][N] -- the drop-in for the reference's UT-solve kernels
// (net/kernels/kda_ut_solve.py:525 kernel, :536 kernel_t) -- and the backward
// rule of their custom_vjp (:563 _backward): dB = the sibling solve of dX,
// dA = strict_lower(-dB X^T) (or strict_lower(-X dB^T) for the transposed
// solve).  fp32 arithmetic; a, b, x fp32 or bf16.
//
// One workgroup per (head, 64-column tile of B): L (zero-padded to 64 x 64)
// and the B tile go to LDS (all of a thread's loads in flight together),
// T = (I + L)^-1 is formed there (kda_tri.h), and X = T B (or T^T B) runs on
// the fp32 matrix cores.  Padding rows/columns beyond C and N are zero and
// never stored.
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

__device__ __forceinline__ f4 mfma4(float a, float b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// A ROWS x 64 block of a row-major [rows][ld] array (element (r, col0 + i)),
// zero outside rows < nr and columns < nc, into LDS [64][kPC]: every load of a
// thread is issued (at a clamped, valid address) before its LDS writes, so the
// loads are in flight together.
template <int DT, bool LOWER>
__device__ __forceinline__ void ut_tile_load(float* dst, const void* src, int64_t base, int ld, int col0, int nr,
                                             int nc) {
  constexpr int PER = kN * kN / kUtThreads;
  float v[PER];
#pragma unroll
  for (int p = 0; p < PER; ++p) {
    const int e = threadIdx.x + kUtThreads * p;
    const int r = e >> 6, i = e & 63;
    const bool ok = r < nr && i < nc && (!LOWER || i < r);
    const int64_t idx = ok ? base + static_cast<int64_t>(r) * ld + col0 + i : base;
    const float x = ut_ld<DT>(src, idx);
    v[p] = ok ? x : 0.f;
  }
#pragma unroll
  for (int p = 0; p < PER; ++p) {
    const int e = threadIdx.x + kUtThreads * p;
    dst[(e >> 6) * kPC + (e & 63)] = v[p];
  }
}

// Forward solve (B = b) or backward rule (B = dX; db written to x, and with
// `da` set, dA from the forward solution `xf`).  X = T B (or T^T B) on the
// fp32 matrix cores: wave w owns row tile w and the four column tiles.
template <int DT, bool TR>
__global__ __launch_bounds__(kUtThreads) void kda_ut_solve_kernel(UtArgs a) {
  __shared__ float sL[kN * kPC], sT[kN * kPC], sB[kN * kPC], tmp[768];
  const int t = threadIdx.x, w = t >> 6, l = t & 63, r = l & 15, gq = l >> 4;
  const int h = blockIdx.x / a.ntiles, tile = blockIdx.x - h * a.ntiles;
  const int j0 = kN * tile;
  const int C = a.C, N = a.N;
  const int64_t abase = static_cast<int64_t>(h) * C * C;
  const int64_t bbase = static_cast<int64_t>(h) * C * N;
  ut_tile_load<DT, true>(sL, a.a, abase, C, 0, C, C);
  ut_tile_load<DT, false>(sB, a.b, bbase, N, j0, C, N - j0);
  __syncthreads();
  invert_unit_lower64<kPC, kUtThreads>(sL, sT, tmp);
  f4 acc[4];
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[q][e] = 0.f;
#pragma unroll 4
  for (int k = 0; k < kN / 4; ++k) {
    const int m = 4 * k + gq;
    const float at = TR ? sT[m * kPC + 16 * w + r] : sT[(16 * w + r) * kPC + m];   // (T or T^T)[c][m]
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[q] = mfma4(at, sB[m * kPC + 16 * q + r], acc[q]);
  }
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int c = 16 * w + 4 * gq + e, col = j0 + 16 * q + r;
      if (c < C && col < N) ut_st<DT>(a.x, bbase + static_cast<int64_t>(c) * N + col, acc[q][e]);
    }
}

// dA[h] = strict_lower(-Y X^T) (TR = false: Y = db, X = forward solution) or
// strict_lower(-X Y^T) (TR = true); one workgroup per head, K = N in tiles of
// 64, on the fp32 matrix cores (wave w: row tile w, four column tiles).
template <int DT, bool TR>
__global__ __launch_bounds__(kUtThreads) void kda_ut_da_kernel(UtArgs a) {
  __shared__ float sY[kN * kPC], sX[kN * kPC];
  const int t = threadIdx.x, w = t >> 6, l = t & 63, r = l & 15, gq = l >> 4;
  const int h = blockIdx.x;
  const int C = a.C, N = a.N;
  const int64_t bbase = static_cast<int64_t>(h) * C * N;
  // P = sum_n R[c][n] Q[i][n] with R = Y, Q = X (TR: R = X, Q = Y)
  const void* Rp = TR ? a.xf : a.x;
  const void* Qp = TR ? a.x : a.xf;
  f4 acc[4];
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[q][e] = 0.f;
  for (int n0 = 0; n0 < N; n0 += kN) {
    ut_tile_load<DT, false>(sY, Rp, bbase, N, n0, C, N - n0);
    ut_tile_load<DT, false>(sX, Qp, bbase, N, n0, C, N - n0);
    __syncthreads();
#pragma unroll 4
    for (int k = 0; k < kN / 4; ++k) {
      const int n = 4 * k + gq;
      const float ar = sY[(16 * w + r) * kPC + n];
#pragma unroll
      for (int q = 0; q < 4; ++q) acc[q] = mfma4(ar, sX[(16 * q + r) * kPC + n], acc[q]);
    }
    __syncthreads();
  }
  const int64_t abase = static_cast<int64_t>(h) * C * C;
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int c = 16 * w + 4 * gq + e, col = 16 * q + r;
      if (c < C && col < C) ut_st<DT>(a.da, abase + static_cast<int64_t>(c) * C + col, (col < c) ? -acc[q][e] : 0.f);
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
