// (I + L)^-1 of a strictly lower-triangular 64 x 64 fp32 matrix in LDS, by one
// workgroup: the four diagonal 16 x 16 blocks by forward substitution (one
// column per thread, in registers), then the off-diagonal blocks by the
// blocked recurrence T_Rs = -T_RR sum_{j=s}^{R-1} L_Rj T_js, block row by
// block row, on the fp32 matrix cores (exact fp32 products).  Used by the
// backward's prep kernel and the standalone solve.
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
  // Off-diagonal blocks on the fp32 matrix cores, one block T_Rs per wave
  // (wave s, s < R): X = sum_{j=s}^{R-1} L_Rj T_js, through the wave's 16 x 16
  // of tmp into the B layout, then T_Rs = -T_RR X.  Lane (r = l & 15,
  // gq = l >> 4) supplies A[r][4k + gq] and B[4k + gq][r] and holds rows
  // 4 gq + e, column r of the result.
  const int wv = t >> 6, l = t & 63, r = l & 15, gq = l >> 4;
  for (int R = 1; R < 4; ++R) {
    if (wv < R) {
      const int sb = wv;
      float* X = tmp + 256 * sb;
      typedef float f4_ __attribute__((ext_vector_type(4)));
      f4_ acc = {0.f, 0.f, 0.f, 0.f};
      for (int j = sb; j < R; ++j) {
#pragma unroll
        for (int k = 0; k < 4; ++k)
          acc = __builtin_amdgcn_mfma_f32_16x16x4f32(sL[(16 * R + r) * PC + 16 * j + 4 * k + gq],
                                                     sT[(16 * j + 4 * k + gq) * PC + 16 * sb + r], acc, 0, 0, 0);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) X[(4 * gq + e) * 16 + r] = acc[e];
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");
      f4_ out = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < 4; ++k)
        out = __builtin_amdgcn_mfma_f32_16x16x4f32(sT[(16 * R + r) * PC + 16 * R + 4 * k + gq],
                                                   X[(4 * k + gq) * 16 + r], out, 0, 0, 0);
#pragma unroll
      for (int e = 0; e < 4; ++e) sT[(16 * R + 4 * gq + e) * PC + 16 * sb + r] = -out[e];
    }
    __syncthreads();
  }
}

}  // namespace kda
