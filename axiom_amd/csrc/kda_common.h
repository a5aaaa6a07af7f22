// Shared device helpers for the KDA kernels (gfx950 / CDNA4 only).
//
// Fragment conventions used by every kernel in this library (64-lane waves):
//   lane l, row-in-tile r = l & 15, lane group gq = l >> 4 (0..3).
//   * MFMA 16x16x32 (f16/bf16): lane holds A[r][k-slots of group gq] (8 values)
//     and B[k-slots of group gq][r]; D (4 fp32) holds rows 4*gq+i, column r.
//   * MFMA 16x16x16 (f16): lane holds A[r][4*gq .. 4*gq+3] and
//     B[4*gq .. 4*gq+3][r]; same D layout.
//   * fp32 "exact" mode replaces one 16x16x32 by eight 16x16x4f32 MFMAs on the
//     same registers (slot e of every lane group forms one K=4 step), so the
//     register layouts are identical in both precisions.
//   * Channel slots.  Inside a 32-wide K step j, slot (gq, e), e = 0..7, carries
//     channel 32*j + 4*gq + (e & 3) + 16*(e >> 2).  With this order the D
//     layouts of two 16x16 tiles (rows 4*gq+i of tile 2j and of tile 2j+1) are
//     exactly the A fragment of one 16x16x32 MFMA, so kernels can hand results
//     to each other through HBM in fragment order with no transpose.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <hip/hip_bf16.h>
#include <stdint.h>

namespace kda {

typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef __bf16 b8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16;

// Cache policy of a direct global->LDS copy (the aux operand of
// __builtin_amdgcn_global_load_lds): non-temporal, for data read once and
// not again by this launch (the copy does not keep the lines in L2, where
// they would displace lines other workgroups still read).
constexpr int kCpolStream = 2;

constexpr float kLog2e = 1.4426950408889634f;

// ----------------------------------------------------------------------------
// element conversions
// ----------------------------------------------------------------------------
__device__ __forceinline__ float bf16_to_f32(u16 b) {
  return __uint_as_float(static_cast<uint32_t>(b) << 16);
}
__device__ __forceinline__ float f16bits_to_f32(u16 b) {
  _Float16 h;
  __builtin_memcpy(&h, &b, 2);
  return static_cast<float>(h);
}
// round-to-nearest-even fp32 -> bf16 bits (finite inputs)
__device__ __forceinline__ u16 f32_to_bf16_bits(float x) {
  uint32_t u = __float_as_uint(x);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return static_cast<u16>(u >> 16);
}

// Input element types: 0 = fp32, 1 = bf16, 2 = fp16.
template <int DT> struct InT;
template <> struct InT<0> { typedef float t; };
template <> struct InT<1> { typedef u16 t; };
template <> struct InT<2> { typedef u16 t; };

template <int DT>
__device__ __forceinline__ float ld1(const void* p, int64_t i) {
  if constexpr (DT == 0) return static_cast<const float*>(p)[i];
  else if constexpr (DT == 1) return bf16_to_f32(static_cast<const u16*>(p)[i]);
  else return f16bits_to_f32(static_cast<const u16*>(p)[i]);
}

// Four packed 16-bit elements (DT 1 = bf16, 2 = fp16) to fp32.
template <int DT>
__device__ __forceinline__ f4 unpack4(uint2 w) {
  f4 r;
  if constexpr (DT == 1) {
    r[0] = __uint_as_float(w.x << 16);
    r[1] = __uint_as_float(w.x & 0xFFFF0000u);
    r[2] = __uint_as_float(w.y << 16);
    r[3] = __uint_as_float(w.y & 0xFFFF0000u);
  } else {
    r[0] = f16bits_to_f32(static_cast<u16>(w.x & 0xFFFFu));
    r[1] = f16bits_to_f32(static_cast<u16>(w.x >> 16));
    r[2] = f16bits_to_f32(static_cast<u16>(w.y & 0xFFFFu));
    r[3] = f16bits_to_f32(static_cast<u16>(w.y >> 16));
  }
  return r;
}

// Four consecutive elements starting at element index i (i multiple of 4).
template <int DT>
__device__ __forceinline__ f4 ld4(const void* p, int64_t i) {
  if constexpr (DT == 0) {
    return *reinterpret_cast<const f4*>(static_cast<const float*>(p) + i);
  } else {
    return unpack4<DT>(*reinterpret_cast<const uint2*>(static_cast<const u16*>(p) + i));
  }
}

// ----------------------------------------------------------------------------
// operand precision: fast (fp16 operands) or exact (fp32 operands)
// ----------------------------------------------------------------------------
template <bool EXACT> struct Prec;
template <> struct Prec<false> {
  typedef _Float16 st;  // storage / operand element
  typedef h8 v8;
  typedef h4 v4;
};
template <> struct Prec<true> {
  typedef float st;
  typedef f8 v8;
  typedef f4 v4;
};

template <bool EXACT>
__device__ __forceinline__ typename Prec<EXACT>::v8 cvt8(const f8& x) {
  if constexpr (EXACT) {
    return x;
  } else {
    h8 r;
#pragma unroll
    for (int i = 0; i < 8; ++i) r[i] = static_cast<_Float16>(x[i]);
    return r;
  }
}
template <bool EXACT>
__device__ __forceinline__ typename Prec<EXACT>::v4 cvt4(const f4& x) {
  if constexpr (EXACT) {
    return x;
  } else {
    h4 r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = static_cast<_Float16>(x[i]);
    return r;
  }
}

// ----------------------------------------------------------------------------
// MFMA wrappers
// ----------------------------------------------------------------------------
__device__ __forceinline__ f4 mma32(f4 acc, h8 a, h8 b) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc, 0, 0, 0);
}
__device__ __forceinline__ f4 mma32(f4 acc, const f8& a, const f8& b) {
#pragma unroll
  for (int e = 0; e < 8; ++e) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[e], b[e], acc, 0, 0, 0);
  return acc;
}
__device__ __forceinline__ f4 mma32_bf16(f4 acc, b8 a, b8 b) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
}
// x = hi + lo with both halves bf16 (hi = x rounded to nearest even)
__device__ __forceinline__ void split_bf16(const f8& x, b8& hi, b8& lo) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const __bf16 h = static_cast<__bf16>(x[e]);
    hi[e] = h;
    lo[e] = static_cast<__bf16>(x[e] - static_cast<float>(h));
  }
}
__device__ __forceinline__ f4 mma16(f4 acc, h4 a, h4 b) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, acc, 0, 0, 0);
}
__device__ __forceinline__ f4 mma16(f4 acc, const f4& a, const f4& b) {
#pragma unroll
  for (int e = 0; e < 4; ++e) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[e], b[e], acc, 0, 0, 0);
  return acc;
}

// ----------------------------------------------------------------------------
// DPP helpers inside 16-lane rows
// ----------------------------------------------------------------------------
// Value of lane (row_base + N) of this lane's 16-lane row.
template <int N>
__device__ __forceinline__ float row_bcast(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
      0, __builtin_bit_cast(int, x), 0x150 + N, 0xF, 0xF, false));
}
// Value of lane (lane - N) in this 16-lane row, 0 for the first N lanes.
template <int N>
__device__ __forceinline__ float row_shr(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
      0, __builtin_bit_cast(int, x), 0x110 + N, 0xF, 0xF, false));
}
// Inclusive prefix sum over the 16 lanes of each DPP row.
__device__ __forceinline__ float row_scan16(float x) {
  x += row_shr<1>(x);
  x += row_shr<2>(x);
  x += row_shr<4>(x);
  x += row_shr<8>(x);
  return x;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// s_waitcnt vmcnt(0), other counters untouched (gfx9 encoding).  Direct
// global->LDS loads are not tracked by the compiler's own waits, so code that
// reads what they wrote waits with this (then orders its LDS reads after it).
__device__ __forceinline__ void wait_vmem_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }
// 8-byte LDS read issued by inline assembly.  The compiler does not see it as
// an LDS access, so it does not make it wait for every outstanding direct
// global->LDS copy of the wave (vmcnt(0)), which it does before each LDS read
// it does see; the caller waits for the copies it needs with wait_vmem<N>()
// first and calls lds_settle() before using the values.
__device__ __forceinline__ uint2 ds_read_b64_raw(const void* p) {
  uint2 v;
  const unsigned addr = static_cast<unsigned>(reinterpret_cast<uintptr_t>(p));
  asm volatile("ds_read_b64 %0, %1" : "=v"(v) : "v"(addr));
  return v;
}
// 16-, 4- and 2-byte forms of the same (the 2-byte read zero-extends), and
// LDS writes the compiler does not see either (it would otherwise wait for
// every outstanding direct copy before them too).
__device__ __forceinline__ u32x4 ds_read_b128_raw(const void* p) {
  u32x4 v;
  const unsigned addr = static_cast<unsigned>(reinterpret_cast<uintptr_t>(p));
  asm volatile("ds_read_b128 %0, %1" : "=v"(v) : "v"(addr));
  return v;
}
__device__ __forceinline__ unsigned ds_read_b32_raw(const void* p) {
  unsigned v;
  const unsigned addr = static_cast<unsigned>(reinterpret_cast<uintptr_t>(p));
  asm volatile("ds_read_b32 %0, %1" : "=v"(v) : "v"(addr));
  return v;
}
__device__ __forceinline__ unsigned ds_read_u16_raw(const void* p) {
  unsigned v;
  const unsigned addr = static_cast<unsigned>(reinterpret_cast<uintptr_t>(p));
  asm volatile("ds_read_u16 %0, %1" : "=v"(v) : "v"(addr));
  return v;
}
__device__ __forceinline__ void ds_write_b32_raw(void* p, unsigned v) {
  const unsigned addr = static_cast<unsigned>(reinterpret_cast<uintptr_t>(p));
  asm volatile("ds_write_b32 %0, %1" : : "v"(addr), "v"(v) : "memory");
}
__device__ __forceinline__ void ds_write_b16_raw(void* p, unsigned v) {
  const unsigned addr = static_cast<unsigned>(reinterpret_cast<uintptr_t>(p));
  asm volatile("ds_write_b16 %0, %1" : : "v"(addr), "v"(v) : "memory");
}
// Waits for all outstanding LDS reads and ties the values to the wait, so no
// use of them is scheduled before it.
template <int N>
__device__ __forceinline__ void lds_settle(uint2 (&v)[N]) {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
  for (int i = 0; i < N; ++i) asm volatile("" : "+v"(v[i]));
}
template <int N>
__device__ __forceinline__ void lds_settle(u32x4 (&v)[N]) {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
  for (int i = 0; i < N; ++i) asm volatile("" : "+v"(v[i]));
}
template <int N>
__device__ __forceinline__ void lds_settle(unsigned (&v)[N]) {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
  for (int i = 0; i < N; ++i) asm volatile("" : "+v"(v[i]));
}

// The layer's elementwise pieces, each defined once so the fused and the
// standalone prologue round alike.  Hardware reciprocal and square root
// (1 ulp) rather than the correctly rounded sequences (12 and 20 instructions).
// 1 / (1 + e^-x): the logistic function of the swish and the output gate
__device__ __forceinline__ float sigmoid_f32(float x) { return __builtin_amdgcn_rcpf(1.f + __expf(-x)); }
// 1 / (sqrt(ss) + 1e-12): the L2 normalisation of a row with sum of squares ss
__device__ __forceinline__ float inv_l2_f32(float ss) {
  return __builtin_amdgcn_rcpf(__builtin_amdgcn_sqrtf(ss) + 1e-12f);
}
// two fp32 -> packed bf16 (round to nearest even, one instruction on gfx950)
typedef float f2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ unsigned pack_bf16x2(float lo, float hi) {
  const f2v v = {lo, hi};
  return __builtin_bit_cast(unsigned, __builtin_convertvector(v, bf2v));
}
__device__ __forceinline__ u16 cvt_bf16(float x) { return __builtin_bit_cast(u16, static_cast<__bf16>(x)); }

// Totals over the 64 lanes of a wavefront of 16 per-lane partial sums (row
// r's partial in ss[r]), as wave-uniform values.  A reduce-scatter over lane
// distances 32, 16, 8, 4 leaves lane l with row 8 b5 + 4 b4 + 2 b3 + b2 (its
// lane bits), two butterfly steps finish it, and each row's total is read from
// a lane holding it.  Every partial formed is the one an xor-butterfly sum
// over distances 32, 16, .., 1 forms, so each total equals that sum bit for bit.
// The reduce-scatter part alone: lane l ends with the total of row
// rowsum16_row(l); a per-row function of the totals can then be evaluated once
// per lane (one instruction for all 16 rows) and read back with readlane.
__device__ __forceinline__ float wave_rowsums16_lanes(const float (&ss)[16]) {
  const int l = __lane_id();
  const bool b5 = (l & 32) != 0, b4 = (l & 16) != 0, b3 = (l & 8) != 0, b2 = (l & 4) != 0;
  float v8[8], v4[4], v2[2];
#pragma unroll
  for (int j = 0; j < 8; ++j) v8[j] = (b5 ? ss[8 + j] : ss[j]) + __shfl_xor(b5 ? ss[j] : ss[8 + j], 32, 64);
#pragma unroll
  for (int j = 0; j < 4; ++j) v4[j] = (b4 ? v8[4 + j] : v8[j]) + __shfl_xor(b4 ? v8[j] : v8[4 + j], 16, 64);
#pragma unroll
  for (int j = 0; j < 2; ++j) v2[j] = (b3 ? v4[2 + j] : v4[j]) + __shfl_xor(b3 ? v4[j] : v4[2 + j], 8, 64);
  float v1 = (b2 ? v2[1] : v2[0]) + __shfl_xor(b2 ? v2[0] : v2[1], 4, 64);
  v1 += __shfl_xor(v1, 2, 64);
  v1 += __shfl_xor(v1, 1, 64);
  return v1;
}
// a lane that holds row r's total after wave_rowsums16_lanes
__device__ __forceinline__ constexpr int rowsum16_lane(int r) {
  return 32 * ((r >> 3) & 1) + 16 * ((r >> 2) & 1) + 8 * ((r >> 1) & 1) + 4 * (r & 1);
}
__device__ __forceinline__ float readlane_f32(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}
__device__ __forceinline__ void wave_rowsums16(const float (&ss)[16], float (&tot)[16]) {
  const float v1 = wave_rowsums16_lanes(ss);
#pragma unroll
  for (int r = 0; r < 16; ++r) tot[r] = readlane_f32(v1, rowsum16_lane(r));
}
// s_waitcnt vmcnt(N): all but the N most recently issued memory operations done
template <int N>
__device__ __forceinline__ void wait_vmem() {
  static_assert(N >= 0 && N < 16, "vmcnt field (low 4 bits)");
  __builtin_amdgcn_s_waitcnt(0x0F70 | N);
}

// Workgroup barrier that orders LDS only.  __syncthreads() also releases
// global memory, which makes every wave wait for its outstanding global loads
// (prefetches) and stores at each barrier; the kernels here never communicate
// through global memory inside a workgroup phase, so they use this one.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// channel carried by slot (gq, e) of 32-wide K step j
__device__ __forceinline__ int slot_channel(int j, int gq, int e) {
  return 32 * j + 4 * gq + (e & 3) + 16 * (e >> 2);
}

}  // namespace kda
