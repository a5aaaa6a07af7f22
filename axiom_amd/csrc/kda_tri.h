// (I + L)^-1 of a strictly lower-triangular 64 x 64 fp32 matrix in LDS, by one
// workgroup: the four diagonal 16 x 16 blocks by forward substitution (one
// column per thread, in registers), then the off-diagonal blocks by the
// blocked recurrence T_Rs = -T_RR sum_{j=s}^{R-1} L_Rj T_js, block row by
// block row.  Used by the backward's prep kernel and the standalone solve.
#pragma once

#include <hip/hip_runtime.h>

namespace kda {

// sL, sT: [64][PC] (PC >= 64); tmp: >= 768 floats of LDS.  L's diagonal and
// upper part are not read.  All NTH threads of the workgroup call it; it
// ends with a barrier, so sT is readable by every thread on return.
template <int PC, int NTH>
__device__ __forceinline__ void invert_unit_lower64(const float* sL, float* sT, float* tmp) {
  const int t = threadIdx.x;
  for (int e = t; e < 64 * 64; e += NTH) {
    const int c = e >> 6, i = e & 63;
    sT[c * PC + i] = 0.f;
  }
  __syncthreads();
  if (t < 64) {
    // column j of the block's inverse: x_i = [i == j] - sum_{m<i} L_im x_m
    // (x_m = 0 for m < j, so the sums may run over all m < i)
    const int R = t >> 4, j = t & 15, a0 = 16 * R;
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float acc = 0.f;
#pragma unroll
      for (int m = 0; m < i; ++m) acc = fmaf(sL[(a0 + i) * PC + a0 + m], x[m], acc);
      x[i] = (i < j) ? 0.f : ((i == j) ? 1.f : -acc);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) sT[(a0 + i) * PC + a0 + j] = x[i];
  }
  __syncthreads();
  for (int R = 1; R < 4; ++R) {
    // X_s = sum_{j=s}^{R-1} L_Rj T_js (s < R) into tmp, then T_Rs = -T_RR X_s
    for (int e = t; e < 256 * R; e += NTH) {
      const int s = e >> 8, rr = (e >> 4) & 15, cc = e & 15;
      float acc = 0.f;
      for (int m = 16 * s; m < 16 * R; ++m) acc = fmaf(sL[(16 * R + rr) * PC + m], sT[m * PC + 16 * s + cc], acc);
      tmp[s * 256 + rr * 16 + cc] = acc;
    }
    __syncthreads();
    for (int e = t; e < 256 * R; e += NTH) {
      const int s = e >> 8, rr = (e >> 4) & 15, cc = e & 15;
      float acc = 0.f;
#pragma unroll
      for (int m = 0; m < 16; ++m) acc = fmaf(sT[(16 * R + rr) * PC + 16 * R + m], tmp[s * 256 + m * 16 + cc], acc);
      sT[(16 * R + rr) * PC + 16 * s + cc] = -acc;
    }
    __syncthreads();
  }
}

}  // namespace kda
