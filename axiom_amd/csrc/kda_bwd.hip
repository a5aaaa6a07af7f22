// Chunked KDA backward (dense [B, T, H, d] inputs), fp32 throughout.
//
// Gradients of o = chunk_fwd(q, k, v, g, beta, h0) and of the final state
// with respect to q, k, v, g (the log decay), beta and h0, following the
// reference's analytic adjoint per chunk (net/kernels/kda_cc_fused_bwd.py:30-55,
// code :139-228) scanned in reverse over the chunks
// (net/kernels/kda_cc_fused_persist.py:794-842, reference_bwd_scan).  Four
// launches:
//   kda_bwd_prep_kernel   one workgroup per chunk-head: in-chunk log2 cumsum G,
//                         gamma*q, lambda*k, gamma_C, Aqk, T = (I+L)^-1, W, U;
//   kda_bwd_fscan_kernel  one workgroup per (chain, 32 value columns): the
//                         forward state scan, keeping every chunk's incoming
//                         state S and its v~ = U - W S;
//   kda_bwd_rscan_kernel  same grid, chunks in reverse: the state cotangent
//                         dS entering each chunk from the right, and
//                         dv~ = (lambda k) dS + Aqk^T do;
//                         dS <- gamma_C dS + (gamma q)^T do - W^T dv~; dh0;
//   kda_bwd_chunk_kernel  one workgroup per chunk-head: the rest of the adjoint
//                         (dY, dgq, dW, the two transposed solves, dL, dAqk, the
//                         score adjoints, the cumsum adjoint) and the outputs.
// Every matrix product is an LDS-tiled fp32 FMA loop (each of the 256 threads
// owns rows r0 + 16i and columns c0 + 16j of the product); decay factors of
// off-diagonal 16-row tiles are anchored at the row tile's first row
// (2^(G_c - G_a) * 2^(G_a - G_i), both <= 1), diagonal tiles use
// 2^(G_c - G_i) directly.  Workspace arrays are fp32, row-major, per
// chunk-head ch = (b * NT + n) * H + h.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "kda_common.h"
#include "kda_internal.h"
#include "kda_tri.h"

namespace kda {
namespace {

constexpr int kC = 64;
constexpr int kThreads = 256;
// The per-chunk adjoint runs 512 threads (two waves per SIMD): it is bound by
// latency at one workgroup per CU (its LDS), so the second wave per SIMD hides it.
constexpr int kChunkThreads = 512;
// Scan workgroups likewise: one per (chain, 32-column slice), 512 threads, one
// state column per thread.
constexpr int kScanThreads = 512;
// The prep kernel likewise (the channel sums of a score tile pair split over
// the two halves of the workgroup).
constexpr int kPrepThreads = 512;

__device__ __forceinline__ float ex2(float x) { return __builtin_amdgcn_exp2f(x); }

template <int D>
struct BwdDims {
  static constexpr int P = D + 1;     // LDS pitch of [rows][D] arrays
  static constexpr int PC = kC + 1;   // LDS pitch of [rows][64] arrays
  static constexpr int NJ = D / 16;   // columns per thread of a [64][D] product
};

// Token row of chunk row c (dense layout) and whether it exists.
struct ChunkRows {
  int64_t row0;   // b * T + n * 64
  int len;        // valid rows of this chunk
};

__device__ __forceinline__ ChunkRows chunk_rows(const BwdArgs& a, int u) {
  const int b = u / a.NT, n = u - b * a.NT;
  ChunkRows r;
  r.row0 = static_cast<int64_t>(b) * a.T + static_cast<int64_t>(n) * kC;
  r.len = min(kC, a.T - n * kC);
  return r;
}

// ROWS x COLS block of a row-major fp32 array (row stride src_ld floats,
// first column col0) into LDS rows of pitch PITCH.  All of a thread's 16-byte
// loads are issued before its LDS writes, so they are in flight together.
// The two halves of lds_load: the loads into registers (a thread's share,
// Tile::PER 16-byte pieces) and the LDS writes.  Split, a scan kernel issues
// the next chunk's loads before the current chunk's arithmetic.
template <int ROWS, int COLS, int NTH = kThreads>
struct Tile {
  static constexpr int V = COLS / 4;
  static constexpr int N = ROWS * V;
  static constexpr int PER = (N + NTH - 1) / NTH;
  static_assert(COLS % 4 == 0, "16-byte loads");
  float4 r[PER];
  __device__ __forceinline__ void fetch(const float* src, int src_ld, int col0) {
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int e = threadIdx.x + p * NTH;
      if (N % NTH == 0 || e < N) {
        const int row = e / V, c4 = e - row * V;
        r[p] = *reinterpret_cast<const float4*>(src + static_cast<int64_t>(row) * src_ld + col0 + 4 * c4);
      }
    }
  }
  template <int PITCH>
  __device__ __forceinline__ void put(float* dst) const {
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int e = threadIdx.x + p * NTH;
      if (N % NTH == 0 || e < N) {
        const int row = e / V, c4 = e - row * V;
        float* d = dst + row * PITCH + 4 * c4;
        d[0] = r[p].x;
        d[1] = r[p].y;
        d[2] = r[p].z;
        d[3] = r[p].w;
      }
    }
  }
};

template <int ROWS, int COLS, int PITCH, int NTH = kThreads>
__device__ __forceinline__ void lds_load(float* dst, const float* src, int src_ld, int col0) {
  Tile<ROWS, COLS, NTH> t;
  t.fetch(src, src_ld, col0);
  t.template put<PITCH>(dst);
}

// Workgroup -> (chain, 32-column slice) of the scan kernels: the NS slices
// of a chain on one XCD (workgroup x runs on XCD x % 8), so the operands all
// of them read come from that XCD's L2.  Grid: ceil(chains / 8) * 8 * NS.
template <int NS>
__device__ __forceinline__ bool scan_slot(int nchains, int& chain, int& split) {
  const int x = blockIdx.x, xcd = x & 7, kk = x >> 3;
  const int slot = kk / NS;
  split = kk - slot * NS;
  chain = slot * 8 + xcd;
  return chain < nchains;
}

// Eight consecutive elements of an input tensor (DT 0 fp32, 1 bf16, 2 fp16)
// as fp32.
template <int DT>
__device__ __forceinline__ void ld8(const void* p, int64_t i, float (&o)[8]) {
  if constexpr (DT == 0) {
    const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + i);
    const float4 b = *reinterpret_cast<const float4*>(static_cast<const float*>(p) + i + 4);
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
    o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
  } else {
    const uint4 w = *reinterpret_cast<const uint4*>(static_cast<const u16*>(p) + i);
    const f4 lo = unpack4<DT>(make_uint2(w.x, w.y)), hi = unpack4<DT>(make_uint2(w.z, w.w));
#pragma unroll
    for (int e = 0; e < 4; ++e) { o[e] = lo[e]; o[4 + e] = hi[e]; }
  }
}

// Columns [col0, col0 + COLS) of the 64 rows of a chunk of a token-major
// input tensor [*, H, D] (rows past `len` read as zero), times mul, into LDS
// rows of pitch PITCH.  Loads issued together, 8 elements per load.
template <int DT, int D, int COLS, int PITCH, int NTH = kThreads>
__device__ __forceinline__ void lds_load_in(float* dst, const void* src, int64_t row0, int len, int H, int h,
                                            int col0, float mul) {
  constexpr int V = COLS / 8;
  constexpr int N = kC * V;
  constexpr int PER = (N + NTH - 1) / NTH;
  static_assert(COLS % 8 == 0, "8-element loads");
  float tmp[PER][8];
#pragma unroll
  for (int p = 0; p < PER; ++p) {
    const int e = threadIdx.x + p * NTH;
    const int r = e / V, c8 = e - r * V;
#pragma unroll
    for (int x = 0; x < 8; ++x) tmp[p][x] = 0.f;
    if ((N % NTH == 0 || e < N) && r < len) ld8<DT>(src, ((row0 + r) * H + h) * D + col0 + 8 * c8, tmp[p]);
  }
#pragma unroll
  for (int p = 0; p < PER; ++p) {
    const int e = threadIdx.x + p * NTH;
    if (N % NTH == 0 || e < N) {
      const int r = e / V, c8 = e - r * V;
#pragma unroll
      for (int x = 0; x < 8; ++x) dst[r * PITCH + 8 * c8 + x] = tmp[p][x] * mul;
    }
  }
}

// ---------------------------------------------------------------------------
// prep: G, gamma*q, lambda*k, gamma_C, Aqk, T, W, U of one chunk-head
// ---------------------------------------------------------------------------
template <int D, int DTQ, int DTG>
__global__ __launch_bounds__(kPrepThreads) void kda_bwd_prep_kernel(BwdArgs a) {
  typedef BwdDims<D> BD;
  constexpr int P = BD::P, PC = BD::PC;
  __shared__ float sQ[kC * P], sK[kC * P], sG[kC * P];
  __shared__ float sL[kC * PC], sT[kC * PC];
  __shared__ float sX0[16 * P], sX1[16 * P], sKf[16 * P];
  __shared__ float sB[kC];
  __shared__ float sRed[2 * 256];   // the second half's partial sums of a tile pair
  constexpr int NTH = kPrepThreads;
  const int t = threadIdx.x;
  const int H = a.H;
  const int u = blockIdx.x / H, h = blockIdx.x - u * H;
  const ChunkRows cr = chunk_rows(a, u);
  const int64_t ch = static_cast<int64_t>(u) * H + h;

  lds_load_in<DTQ, D, D, P, NTH>(sQ, a.q, cr.row0, cr.len, H, h, 0, a.scale);
  lds_load_in<DTQ, D, D, P, NTH>(sK, a.k, cr.row0, cr.len, H, h, 0, 1.f);
  lds_load_in<DTG, D, D, P, NTH>(sG, a.g, cr.row0, cr.len, H, h, 0, 1.f);
  if (t < kC) sB[t] = (t < cr.len) ? ld1<DTG>(a.beta, (cr.row0 + t) * H + h) : 0.f;
  __syncthreads();
  // in-chunk inclusive cumsum of g, in log2 units
  if (t < D) {
    float col[kC];
#pragma unroll
    for (int c = 0; c < kC; ++c) col[c] = sG[c * P + t];
    float acc = 0.f;
#pragma unroll
    for (int c = 0; c < kC; ++c) {
      acc += col[c];
      sG[c * P + t] = acc * kLog2e;
    }
  }
  __syncthreads();
  {
    float* GL = a.GL + ch * kC * D;
    float* QG = a.QG + ch * kC * D;
    float* KL = a.KL + ch * kC * D;
    for (int e = t; e < kC * D; e += NTH) {
      const int c = e / D, d = e - c * D;
      const float gl = sG[c * P + d];
      const float glast = sG[(kC - 1) * P + d];
      GL[e] = gl;
      QG[e] = ex2(gl) * sQ[c * P + d];
      KL[e] = ex2(glast - gl) * sK[c * P + d];
    }
    if (t < D) a.GCV[ch * D + t] = ex2(sG[(kC - 1) * P + t]);
  }

  // scores: Aqk (c >= i) straight to the workspace, L = beta_c Akk (c > i) to LDS
  float* AQ = a.AQ + ch * kC * kC;
  // output (r, i16) of a 16 x 16 tile pair; the two halves of the workgroup
  // sum over the two halves of the channels and add up through sRed
  const int t2 = t & 255, half = t >> 8;
  const int r = t2 >> 4, i16 = t2 & 15;
  const int d0 = half * (D / 2);
  for (int R = 0; R < 4; ++R) {
    const int a0 = 16 * R;
    // row operands of tile R with the factor 2^(G_c - G_a)
    for (int e = t; e < 16 * D; e += NTH) {
      const int rr = e / D, d = e - rr * D;
      const float fr = ex2(sG[(a0 + rr) * P + d] - sG[a0 * P + d]);
      sX0[rr * P + d] = sQ[(a0 + rr) * P + d] * fr;
      sX1[rr * P + d] = sK[(a0 + rr) * P + d] * sB[a0 + rr] * fr;
    }
    for (int s = 0; s < R; ++s) {
      __syncthreads();  // sX0/sX1 written; previous sKf readers done
      for (int e = t; e < 16 * D; e += NTH) {
        const int ii = e / D, d = e - ii * D;
        sKf[ii * P + d] = sK[(16 * s + ii) * P + d] * ex2(sG[a0 * P + d] - sG[(16 * s + ii) * P + d]);
      }
      __syncthreads();
      float accA = 0.f, accL = 0.f;
      #pragma unroll 4
      for (int d = d0; d < d0 + D / 2; ++d) {
        const float kf = sKf[i16 * P + d];
        accA = fmaf(sX0[r * P + d], kf, accA);
        accL = fmaf(sX1[r * P + d], kf, accL);
      }
      if (half) { sRed[t2] = accA; sRed[256 + t2] = accL; }
      __syncthreads();
      if (!half) {
        AQ[(a0 + r) * kC + 16 * s + i16] = accA + sRed[t2];
        sL[(a0 + r) * PC + 16 * s + i16] = accL + sRed[256 + t2];
      }
    }
    // diagonal tile, 2^(G_c - G_i) directly
    {
      const int c = a0 + r, i = a0 + i16;
      float accA = 0.f, accL = 0.f;
      if (i16 <= r) {
        #pragma unroll 4
        for (int d = d0; d < d0 + D / 2; ++d) {
          const float e = ex2(sG[c * P + d] - sG[i * P + d]);
          const float ki = sK[i * P + d] * e;
          accA = fmaf(sQ[c * P + d], ki, accA);
          accL = fmaf(sK[c * P + d], ki, accL);
        }
      }
      __syncthreads();   // the off-diagonal sums have been read out of sRed
      if (half) { sRed[t2] = accA; sRed[256 + t2] = accL; }
      __syncthreads();
      if (!half) {
        AQ[c * kC + i] = accA + sRed[t2];
        sL[c * PC + i] = (i16 < r) ? (accL + sRed[256 + t2]) * sB[c] : 0.f;
        // upper triangle of the row band: zero
        for (int s = R + 1; s < 4; ++s) {
          AQ[c * kC + 16 * s + i16] = 0.f;
          sL[c * PC + 16 * s + i16] = 0.f;
        }
      }
    }
    __syncthreads();  // sX0/sX1 reused by the next row tile
  }

  // T = (I + L)^-1
  invert_unit_lower64<PC, NTH>(sL, sT, sX0);
  {
    float* TM = a.TM + ch * kC * kC;
    for (int e = t; e < kC * kC; e += NTH) {
      const int c = e / kC, i = e - c * kC;
      TM[e] = sT[c * PC + i];
    }
  }
  // W = T (beta gamma k), U = T (beta v)
  lds_load_in<DTQ, D, D, P, NTH>(sQ, a.v, cr.row0, cr.len, H, h, 0, 1.f);
  __syncthreads();
  for (int e = t; e < kC * D; e += NTH) {
    const int c = e / D, d = e - c * D;
    sK[c * P + d] *= sB[c] * ex2(sG[c * P + d]);
    sQ[c * P + d] *= sB[c];
  }
  __syncthreads();
  {
    constexpr int TC = NTH / 16;
    constexpr int NJ = D / TC;
    const int rm = t / TC, cn = t % TC;
    float accW[4][NJ], accU[4][NJ];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j) accW[i][j] = accU[i][j] = 0.f;
    #pragma unroll 4
    for (int m = 0; m < kC; ++m) {
      float tv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) tv[i] = sT[(rm + 16 * i) * PC + m];
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const float x = sK[m * P + cn + TC * j], y = sQ[m * P + cn + TC * j];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          accW[i][j] = fmaf(tv[i], x, accW[i][j]);
          accU[i][j] = fmaf(tv[i], y, accU[i][j]);
        }
      }
    }
    float* WM = a.WM + ch * kC * D;
    float* UM = a.UM + ch * kC * D;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        WM[(rm + 16 * i) * D + cn + TC * j] = accW[i][j];
        UM[(rm + 16 * i) * D + cn + TC * j] = accU[i][j];
      }
  }
}

// ---------------------------------------------------------------------------
// The two scans run their products on the fp32 matrix cores
// (v_mfma_f32_16x16x4f32, exact fp32 products): lane (r = l & 15, gq = l >> 4)
// supplies A[r][4s + gq] and B[4s + gq][r] of K step s and holds D rows
// 4 gq + i, column r.  Eight waves per workgroup; the 32-column state slice is
// (D/16) x 2 tiles in accumulators, D/64 tiles per wave; the [64][32] results
// of a chunk are 8 tiles, one per wave.  LDS pitches: PW = D + 2 for [64][D]
// operands (row fragments conflict-free, column fragments 2-way), PB = 48 for
// [*][32] B operands, PA = 80 for Aqk read by columns.
// ---------------------------------------------------------------------------
constexpr int kPB = 48;
constexpr int kPA = kC + 16;

__device__ __forceinline__ f4 mfma4(float a, float b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// forward state scan of one (chain, 32-column slice): S_in and v~ per chunk
template <int D>
__global__ __launch_bounds__(kScanThreads) void kda_bwd_fscan_kernel(BwdArgs a) {
  constexpr int PW = D + 2;
  constexpr int NS = D / 32;
  constexpr int NST = D / 64;   // state tiles per wave
  __shared__ float sW[kC * PW], sKL[kC * PW];
  __shared__ float sS[D * kPB], sU[kC * kPB], sV[kC * kPB], sGC[D];
  constexpr int NTH = kScanThreads;
  const int t = threadIdx.x, wv = t >> 6, l = t & 63, r = l & 15, gq = l >> 4;
  const int H = a.H;
  int chain, split;
  if (!scan_slot<NS>(a.B * H, chain, split)) return;   // uniform per workgroup
  const int b = chain / H, h = chain - b * H;
  const int c0 = 32 * split;
  const int mt = wv >> 1, ct = wv & 1;                  // this wave's v~ tile
  int rt[NST], cs[NST];                                 // this wave's state tiles
#pragma unroll
  for (int q = 0; q < NST; ++q) { rt[q] = (wv * NST + q) >> 1; cs[q] = (wv * NST + q) & 1; }
  f4 S[NST];
#pragma unroll
  for (int q = 0; q < NST; ++q)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      S[q][i] = (a.h0 != nullptr)
                    ? a.h0[(static_cast<int64_t>(chain) * D + 16 * rt[q] + 4 * gq + i) * D + c0 + 16 * cs[q] + r]
                    : 0.f;
  // chunk n's W, lambda*k and U slice are loaded into registers during
  // chunk n-1's arithmetic
  Tile<kC, D, NTH> tW, tK;
  Tile<kC, 32, NTH> tU;
  auto fetch = [&](int n) {
    const int64_t ch = (static_cast<int64_t>(b) * a.NT + n) * H + h;
    tW.fetch(a.WM + ch * kC * D, D, 0);
    tK.fetch(a.KL + ch * kC * D, D, 0);
    tU.fetch(a.UM + ch * kC * D, D, c0);
  };
  if (a.NT > 0) fetch(0);
  for (int n = 0; n < a.NT; ++n) {
    const int64_t ch = (static_cast<int64_t>(b) * a.NT + n) * H + h;
    float* SI = a.SI + ch * D * D;
#pragma unroll
    for (int q = 0; q < NST; ++q)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 16 * rt[q] + 4 * gq + i, col = 16 * cs[q] + r;
        SI[row * D + c0 + col] = S[q][i];
        sS[row * kPB + col] = S[q][i];
      }
    tW.template put<PW>(sW);
    tK.template put<PW>(sKL);
    tU.template put<kPB>(sU);
    if (t < D) sGC[t] = a.GCV[ch * D + t];
    if (n + 1 < a.NT) fetch(n + 1);
    __syncthreads();
    // v~ = U - W S (two accumulation chains over K = D)
    {
      f4 acc0, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < 4; ++i) acc0[i] = sU[(16 * mt + 4 * gq + i) * kPB + 16 * ct + r];
#pragma unroll 8
      for (int k = 0; k < D / 4; k += 2) {
        acc0 = mfma4(-sW[(16 * mt + r) * PW + 4 * k + gq], sS[(4 * k + gq) * kPB + 16 * ct + r], acc0);
        acc1 = mfma4(-sW[(16 * mt + r) * PW + 4 * k + 4 + gq], sS[(4 * k + 4 + gq) * kPB + 16 * ct + r], acc1);
      }
      float* VT = a.VT + ch * kC * D;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 16 * mt + 4 * gq + i, col = 16 * ct + r;
        const float v = acc0[i] + acc1[i];
        sV[row * kPB + col] = v;
        VT[row * D + c0 + col] = v;
      }
    }
    __syncthreads();
    // S <- gamma_C S + (lambda k)^T v~
#pragma unroll
    for (int q = 0; q < NST; ++q)
#pragma unroll
      for (int i = 0; i < 4; ++i) S[q][i] *= sGC[16 * rt[q] + 4 * gq + i];
#pragma unroll 4
    for (int k = 0; k < kC / 4; ++k)
#pragma unroll
      for (int q = 0; q < NST; ++q)
        S[q] = mfma4(sKL[(4 * k + gq) * PW + 16 * rt[q] + r], sV[(4 * k + gq) * kPB + 16 * cs[q] + r], S[q]);
    __syncthreads();
  }
}

// reverse scan of one (chain, 32-column slice): dS per chunk, dv~, dh0
template <int D, int DO>
__global__ __launch_bounds__(kScanThreads) void kda_bwd_rscan_kernel(BwdArgs a) {
  constexpr int PW = D + 2;
  constexpr int NS = D / 32;
  constexpr int NST = D / 64;
  __shared__ float sX[kC * PW], sY[kC * PW], sA[kC * kPA];
  __shared__ float sS[D * kPB], sDo[kC * kPB], sDv[kC * kPB], sGC[D];
  constexpr int NTH = kScanThreads;
  const int t = threadIdx.x, wv = t >> 6, l = t & 63, r = l & 15, gq = l >> 4;
  const int H = a.H;
  int chain, split;
  if (!scan_slot<NS>(a.B * H, chain, split)) return;   // uniform per workgroup
  const int b = chain / H, h = chain - b * H;
  const int c0 = 32 * split;
  const int mt = wv >> 1, ct = wv & 1;
  int rt[NST], cs[NST];
#pragma unroll
  for (int q = 0; q < NST; ++q) { rt[q] = (wv * NST + q) >> 1; cs[q] = (wv * NST + q) & 1; }
  f4 dS[NST];
#pragma unroll
  for (int q = 0; q < NST; ++q)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      dS[q][i] = (a.dht != nullptr)
                     ? a.dht[(static_cast<int64_t>(chain) * D + 16 * rt[q] + 4 * gq + i) * D + c0 + 16 * cs[q] + r]
                     : 0.f;
  // Operands of the two products of a chunk, loaded into registers one
  // product ahead: lambda*k and Aqk (for dv~) during the previous chunk's dS
  // update, gamma*q and W (for dS) during this chunk's dv~.
  Tile<kC, D, NTH> tX, tY;
  Tile<kC, kC, NTH> tA;
  auto fetch_a = [&](int n) {
    const int64_t ch = (static_cast<int64_t>(b) * a.NT + n) * H + h;
    tX.fetch(a.KL + ch * kC * D, D, 0);
    tA.fetch(a.AQ + ch * kC * kC, kC, 0);
  };
  if (a.NT > 0) fetch_a(a.NT - 1);
  for (int n = a.NT - 1; n >= 0; --n) {
    const int u = b * a.NT + n;
    const int64_t ch = static_cast<int64_t>(u) * H + h;
    const ChunkRows cr = chunk_rows(a, u);
    float* DS = a.DS + ch * D * D;
#pragma unroll
    for (int q = 0; q < NST; ++q)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 16 * rt[q] + 4 * gq + i, col = 16 * cs[q] + r;
        DS[row * D + c0 + col] = dS[q][i];
        sS[row * kPB + col] = dS[q][i];
      }
    tX.template put<PW>(sX);
    tA.template put<kPA>(sA);
    lds_load_in<DO, D, 32, kPB, NTH>(sDo, a.dout, cr.row0, cr.len, H, h, c0, 1.f);
    if (t < D) sGC[t] = a.GCV[ch * D + t];
    tX.fetch(a.QG + ch * kC * D, D, 0);
    tY.fetch(a.WM + ch * kC * D, D, 0);
    __syncthreads();
    // dv~ = (lambda k) dS + Aqk^T do
    {
      f4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
      for (int k = 0; k < D / 4; ++k)
        acc0 = mfma4(sX[(16 * mt + r) * PW + 4 * k + gq], sS[(4 * k + gq) * kPB + 16 * ct + r], acc0);
#pragma unroll 8
      for (int k = 0; k < kC / 4; ++k)
        acc1 = mfma4(sA[(4 * k + gq) * kPA + 16 * mt + r], sDo[(4 * k + gq) * kPB + 16 * ct + r], acc1);
      float* DVT = a.DVT + ch * kC * D;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 16 * mt + 4 * gq + i, col = 16 * ct + r;
        const float v = acc0[i] + acc1[i];
        sDv[row * kPB + col] = v;
        DVT[row * D + c0 + col] = v;
      }
    }
    __syncthreads();
    tX.template put<PW>(sX);
    tY.template put<PW>(sY);
    if (n > 0) fetch_a(n - 1);
    __syncthreads();
    // dS <- gamma_C dS + (gamma q)^T do - W^T dv~
#pragma unroll
    for (int q = 0; q < NST; ++q)
#pragma unroll
      for (int i = 0; i < 4; ++i) dS[q][i] *= sGC[16 * rt[q] + 4 * gq + i];
#pragma unroll 4
    for (int k = 0; k < kC / 4; ++k)
#pragma unroll
      for (int q = 0; q < NST; ++q) {
        const int kr = (4 * k + gq) * PW + 16 * rt[q] + r, kb = (4 * k + gq) * kPB + 16 * cs[q] + r;
        dS[q] = mfma4(sX[kr], sDo[kb], dS[q]);
        dS[q] = mfma4(-sY[kr], sDv[kb], dS[q]);
      }
    __syncthreads();
  }
  if (a.dh0 != nullptr) {
#pragma unroll
    for (int q = 0; q < NST; ++q)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        a.dh0[(static_cast<int64_t>(chain) * D + 16 * rt[q] + 4 * gq + i) * D + c0 + 16 * cs[q] + r] = dS[q][i];
  }
}

// ---------------------------------------------------------------------------
// per chunk-head adjoint
// ---------------------------------------------------------------------------
template <int D, int DTQ, int DTG, int DO>
__global__ __launch_bounds__(kChunkThreads) void kda_bwd_chunk_kernel(BwdArgs a) {
  typedef BwdDims<D> BD;
  constexpr int P = BD::P, PC = BD::PC;
  constexpr int NTH = kChunkThreads;
  constexpr int TC = NTH / 16;        // threads per row group: columns cn + TC j
  constexpr int NJ = D / TC;          // columns per thread of a [64][D] product
  constexpr int NJC = kC / TC;        // of a [64][64] product
  constexpr int HW = 64;             // value columns per pass of phase 1
  constexpr int NH = D / HW;
  // phase 4 is the largest: dL, dAqk [64][65]; q, k, G [64][P]; three [16][P]
  constexpr int SMEM_FLOATS = 2 * kC * PC + 3 * kC * P + 3 * 16 * P + kC;
  __shared__ float sm[SMEM_FLOATS];
  const int t = threadIdx.x, rm = t / TC, cn = t % TC;
  const int H = a.H;
  const int u = blockIdx.x / H, h = blockIdx.x - u * H;
  const ChunkRows cr = chunk_rows(a, u);
  const int64_t ch = static_cast<int64_t>(u) * H + h;
  const float* GL = a.GL + ch * kC * D;
  auto in_idx = [&](int c, int d) { return ((cr.row0 + c) * H + h) * D + d; };
  auto ld_q = [&](int c, int d) { return (c < cr.len) ? ld1<DTQ>(a.q, in_idx(c, d)) * a.scale : 0.f; };
  auto ld_k = [&](int c, int d) { return (c < cr.len) ? ld1<DTQ>(a.k, in_idx(c, d)) : 0.f; };
  auto ld_v = [&](int c, int d) { return (c < cr.len) ? ld1<DTQ>(a.v, in_idx(c, d)) : 0.f; };
  auto ld_b = [&](int c) { return (c < cr.len) ? ld1<DTG>(a.beta, (cr.row0 + c) * H + h) : 0.f; };
  // The gradients of q, k and G accumulate in place in dq, dk and dg (dg
  // holds dG until the final reverse cumsum): each thread owns the positions
  // (rm + 16i, cn + 16j) of its row tile i = 0..3, so its own read-modify-
  // writes need no synchronisation; pad rows (c >= len) are never stored
  // (their dG is zero: every term carries a factor q_c or k_c).
  float* const gq_ = a.dq;
  float* const gk_ = a.dk;
  float* const gG_ = a.dg;

  float dbr[4], dzp[NJ];
#pragma unroll
  for (int i = 0; i < 4; ++i) dbr[i] = 0.f;
#pragma unroll
  for (int j = 0; j < NJ; ++j) dzp[j] = 0.f;
  float dgc = 0.f;   // thread t < D: sum_n S[t][n] dS'[t][n]

  // ---- phase 1: dY = v~ dS'^T, dgq = do S^T, dW = -dv~ S^T (K = dv in passes of 64)
  float dW[4][NJ];
  {
    float dY[4][NJ], dgq[4][NJ];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j) dY[i][j] = dgq[i][j] = dW[i][j] = 0.f;
    float* sVt = sm;
    float* sDo = sVt + kC * PC;
    float* sDv = sDo + kC * PC;
    float* sS = sDv + kC * PC;
    float* sDS = sS + D * PC;
    for (int hp = 0; hp < NH; ++hp) {
      const int n0 = HW * hp;
      lds_load<kC, HW, PC, NTH>(sVt, a.VT + ch * kC * D, D, n0);
      lds_load<kC, HW, PC, NTH>(sDv, a.DVT + ch * kC * D, D, n0);
      lds_load<D, HW, PC, NTH>(sS, a.SI + ch * D * D, D, n0);
      lds_load<D, HW, PC, NTH>(sDS, a.DS + ch * D * D, D, n0);
      lds_load_in<DO, D, HW, PC, NTH>(sDo, a.dout, cr.row0, cr.len, H, h, n0, 1.f);
      __syncthreads();
      #pragma unroll 4
      for (int nn = 0; nn < HW; ++nn) {
        float va[4], oa[4], wa[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          va[i] = sVt[(rm + 16 * i) * PC + nn];
          oa[i] = sDo[(rm + 16 * i) * PC + nn];
          wa[i] = sDv[(rm + 16 * i) * PC + nn];
        }
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const float sv = sS[(cn + TC * j) * PC + nn], dsv = sDS[(cn + TC * j) * PC + nn];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            dY[i][j] = fmaf(va[i], dsv, dY[i][j]);
            dgq[i][j] = fmaf(oa[i], sv, dgq[i][j]);
            dW[i][j] = fmaf(-wa[i], sv, dW[i][j]);
          }
        }
      }
      if (t < D) {
        for (int nn = 0; nn < HW; ++nn) dgc = fmaf(sS[t * PC + nn], sDS[t * PC + nn], dgc);
      }
      __syncthreads();
    }
    // dq = dgq gamma; dG = dgq q gamma - dY k lambda; dk = dY lambda.  Each
    // row tile's loads are issued before its stores (the compiler cannot move
    // a load above a store to a pointer it may alias).
    float glast[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) glast[j] = GL[(kC - 1) * D + cn + TC * j];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = rm + 16 * i;
      float gl[NJ], qv[NJ], kv[NJ];
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        gl[j] = GL[c * D + cn + TC * j];
        qv[j] = ld_q(c, cn + TC * j);
        kv[j] = ld_k(c, cn + TC * j);
      }
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int d = cn + TC * j;
        const float gam = ex2(gl[j]), lam = ex2(glast[j] - gl[j]);
        const float dz = dY[i][j] * kv[j] * lam;
        dzp[j] += dz;
        if (c < cr.len) {
          gq_[in_idx(c, d)] = dgq[i][j] * gam * a.scale;
          gk_[in_idx(c, d)] = dY[i][j] * lam;
          gG_[in_idx(c, d)] = dgq[i][j] * qv[j] * gam - dz;
        }
      }
    }
  }

  // ---- phase 2: Yw = T^T dW, Yu = T^T dv~
  float Yw[4][NJ], Yu[4][NJ];
  {
    float* sT = sm;
    float* sX = sT + kC * PC;
    float* sY = sX + kC * P;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j) sX[(rm + 16 * i) * P + cn + TC * j] = dW[i][j];
    lds_load<kC, kC, PC, NTH>(sT, a.TM + ch * kC * kC, kC, 0);
    lds_load<kC, D, P, NTH>(sY, a.DVT + ch * kC * D, D, 0);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j) Yw[i][j] = Yu[i][j] = 0.f;
    #pragma unroll 4
    for (int m = 0; m < kC; ++m) {
      float tv[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) tv[i] = sT[m * PC + rm + 16 * i];
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const float x = sX[m * P + cn + TC * j], y = sY[m * P + cn + TC * j];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          Yw[i][j] = fmaf(tv[i], x, Yw[i][j]);
          Yu[i][j] = fmaf(tv[i], y, Yu[i][j]);
        }
      }
    }
    __syncthreads();
    // dG += Yw k beta gamma; dk += Yw gamma beta; dv = Yu beta; dbeta += Yw gamma k + Yu v
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = rm + 16 * i;
      const bool live = c < cr.len;
      const float bc = ld_b(c);
      float gl[NJ], kv[NJ], vv[NJ], oG[NJ], ok[NJ];
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int d = cn + TC * j;
        gl[j] = GL[c * D + d];
        kv[j] = ld_k(c, d);
        vv[j] = ld_v(c, d);
        oG[j] = live ? gG_[in_idx(c, d)] : 0.f;
        ok[j] = live ? gk_[in_idx(c, d)] : 0.f;
      }
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int d = cn + TC * j;
        const float gam = ex2(gl[j]);
        dbr[i] += Yw[i][j] * gam * kv[j] + Yu[i][j] * vv[j];
        if (live) {
          gG_[in_idx(c, d)] = oG[j] + Yw[i][j] * kv[j] * bc * gam;
          gk_[in_idx(c, d)] = ok[j] + Yw[i][j] * gam * bc;
          a.dv[in_idx(c, d)] = Yu[i][j] * bc;
        }
      }
    }
  }

  // ---- phase 3: dL = strict(-(Yw W^T + Yu U^T)), dAqk = tril(do v~^T)
  float dLr[4][NJC], dAr[4][NJC];   // rows rm + 16i, columns cn + TC j
  {
    float* sX = sm;
    float* sY = sX + kC * P;
    float* sW = sY + kC * P;
    float* sU = sW + kC * P;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        sX[(rm + 16 * i) * P + cn + TC * j] = Yw[i][j];
        sY[(rm + 16 * i) * P + cn + TC * j] = Yu[i][j];
      }
    lds_load<kC, D, P, NTH>(sW, a.WM + ch * kC * D, D, 0);
    lds_load<kC, D, P, NTH>(sU, a.UM + ch * kC * D, D, 0);
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < NJC; ++j) dLr[i][j] = dAr[i][j] = 0.f;
    #pragma unroll 4
    for (int d = 0; d < D; ++d) {
      float yw[4], yu[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        yw[i] = sX[(rm + 16 * i) * P + d];
        yu[i] = sY[(rm + 16 * i) * P + d];
      }
#pragma unroll
      for (int j = 0; j < NJC; ++j) {
        const float w = sW[(cn + TC * j) * P + d], uu = sU[(cn + TC * j) * P + d];
#pragma unroll
        for (int i = 0; i < 4; ++i) dLr[i][j] = fmaf(yw[i], w, fmaf(yu[i], uu, dLr[i][j]));
      }
    }
    __syncthreads();
    // do and v~ into the W / U slots
    lds_load_in<DO, D, D, P, NTH>(sW, a.dout, cr.row0, cr.len, H, h, 0, 1.f);
    lds_load<kC, D, P, NTH>(sU, a.VT + ch * kC * D, D, 0);
    __syncthreads();
    #pragma unroll 4
    for (int d = 0; d < D; ++d) {
      float ov[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) ov[i] = sW[(rm + 16 * i) * P + d];
#pragma unroll
      for (int j = 0; j < NJC; ++j) {
        const float vv = sU[(cn + TC * j) * P + d];
#pragma unroll
        for (int i = 0; i < 4; ++i) dAr[i][j] = fmaf(ov[i], vv, dAr[i][j]);
      }
    }
    __syncthreads();
  }

  // ---- phase 4: score adjoints (Aqk with rows q, columns k; L with rows k beta, columns k)
  {
    float* sDL = sm;
    float* sDA = sDL + kC * PC;
    float* sQ = sDA + kC * PC;
    float* sK = sQ + kC * P;
    float* sG = sK + kC * P;
    float* sXq = sG + kC * P;
    float* sXk = sXq + 16 * P;
    float* sKf = sXk + 16 * P;
    float* sB = sKf + 16 * P;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < NJC; ++j) {
        const int c = rm + 16 * i, ii = cn + TC * j;
        sDL[c * PC + ii] = (ii < c) ? -dLr[i][j] : 0.f;
        sDA[c * PC + ii] = (ii <= c) ? dAr[i][j] : 0.f;
      }
    lds_load_in<DTQ, D, D, P, NTH>(sQ, a.q, cr.row0, cr.len, H, h, 0, a.scale);
    lds_load_in<DTQ, D, D, P, NTH>(sK, a.k, cr.row0, cr.len, H, h, 0, 1.f);
    lds_load<kC, D, P, NTH>(sG, GL, D, 0);
    if (t < kC) sB[t] = ld_b(t);
    __syncthreads();
    for (int R = 0; R < 4; ++R) {
      const int a0 = 16 * R;
      for (int e = t; e < 16 * D; e += NTH) {
        const int rr = e / D, d = e - rr * D;
        const float fr = ex2(sG[(a0 + rr) * P + d] - sG[a0 * P + d]);
        sXq[rr * P + d] = sQ[(a0 + rr) * P + d] * fr;
        sXk[rr * P + d] = sK[(a0 + rr) * P + d] * sB[a0 + rr] * fr;
      }
      float drA[NJ], drK[NJ];   // row c = a0 + rm: factorised part (times 2^(G_c - G_a) at the end)
#pragma unroll
      for (int j = 0; j < NJ; ++j) drA[j] = drK[j] = 0.f;
      const int c = a0 + rm;
      for (int s = 0; s < R; ++s) {
        __syncthreads();
        for (int e = t; e < 16 * D; e += NTH) {
          const int ii = e / D, d = e - ii * D;
          sKf[ii * P + d] = sK[(16 * s + ii) * P + d] * ex2(sG[a0 * P + d] - sG[(16 * s + ii) * P + d]);
        }
        __syncthreads();
        // row side: dr[c] += sum_{i in s} D[c][i] k_i 2^(G_a - G_i)
        #pragma unroll 4
        for (int ii = 0; ii < 16; ++ii) {
          const float da = sDA[c * PC + 16 * s + ii], dl = sDL[c * PC + 16 * s + ii];
#pragma unroll
          for (int j = 0; j < NJ; ++j) {
            const float kf = sKf[ii * P + cn + TC * j];
            drA[j] = fmaf(da, kf, drA[j]);
            drK[j] = fmaf(dl, kf, drK[j]);
          }
        }
        // column side for key row i = 16s + rm: sum_{c' in R} D[c'][i] x_c' 2^(G_c' - G_a), times 2^(G_a - G_i)
        {
          const int i = 16 * s + rm;
          float dcA[NJ], dcK[NJ];
#pragma unroll
          for (int j = 0; j < NJ; ++j) dcA[j] = dcK[j] = 0.f;
          #pragma unroll 4
          for (int rr = 0; rr < 16; ++rr) {
            const float da = sDA[(a0 + rr) * PC + i], dl = sDL[(a0 + rr) * PC + i];
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
              dcA[j] = fmaf(da, sXq[rr * P + cn + TC * j], dcA[j]);
              dcK[j] = fmaf(dl, sXk[rr * P + cn + TC * j], dcK[j]);
            }
          }
          if (i < cr.len) {
            float ok[NJ], oG[NJ];
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
              ok[j] = gk_[in_idx(i, cn + TC * j)];
              oG[j] = gG_[in_idx(i, cn + TC * j)];
            }
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
              const int d = cn + TC * j;
              const float fk = ex2(sG[a0 * P + d] - sG[i * P + d]);
              const float sum = (dcA[j] + dcK[j]) * fk;
              gk_[in_idx(i, d)] = ok[j] + sum;
              gG_[in_idx(i, d)] = oG[j] - sum * sK[i * P + d];
            }
          }
        }
      }
      // diagonal tile and the row-side totals
      {
        const int i = a0 + rm;   // the same row, as a key row of the diagonal tile
        float dbsum = 0.f;
        float oq[NJ], oG[NJ], ok[NJ];
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const bool live = c < cr.len;
          oq[j] = live ? gq_[in_idx(c, cn + TC * j)] : 0.f;
          oG[j] = live ? gG_[in_idx(c, cn + TC * j)] : 0.f;
          ok[j] = live ? gk_[in_idx(c, cn + TC * j)] : 0.f;
        }
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const int d = cn + TC * j;
          const float gc = sG[c * P + d];
          float rA = drA[j] * ex2(gc - sG[a0 * P + d]);
          float rK = drK[j] * ex2(gc - sG[a0 * P + d]);
          float cA = 0.f, cK = 0.f;
          for (int ii = 0; ii <= rm; ++ii) {
            const int ik = a0 + ii;
            const float e = ex2(gc - sG[ik * P + d]);
            const float ke = sK[ik * P + d] * e;
            rA = fmaf(sDA[c * PC + ik], ke, rA);
            rK = fmaf(sDL[c * PC + ik], ke, rK);
          }
          const float gi = sG[i * P + d];
          for (int rr = rm; rr < 16; ++rr) {
            const int cc = a0 + rr;
            const float e = ex2(sG[cc * P + d] - gi);
            cA = fmaf(sDA[cc * PC + i], sQ[cc * P + d] * e, cA);
            cK = fmaf(sDL[cc * PC + i], sK[cc * P + d] * sB[cc] * e, cK);
          }
          const float qv = sQ[c * P + d], kv = sK[c * P + d], bc = sB[c];
          dbsum += rK * kv;
          if (c < cr.len) {
            gq_[in_idx(c, d)] = oq[j] + rA * a.scale;
            gG_[in_idx(c, d)] = oG[j] + rA * qv + rK * kv * bc - (cA + cK) * kv;
            gk_[in_idx(c, d)] = ok[j] + rK * bc + cA + cK;
          }
        }
        // dbr is indexed by the row tile: R is a runtime loop here, so add
        // through the per-row LDS reduction below instead of a register array
        dbr[0] += (R == 0) ? dbsum : 0.f;
        dbr[1] += (R == 1) ? dbsum : 0.f;
        dbr[2] += (R == 2) ? dbsum : 0.f;
        dbr[3] += (R == 3) ? dbsum : 0.f;
      }
      __syncthreads();
    }
  }

  // ---- outputs: dbeta, dg (reverse cumsum of dG plus the G_C terms)
  {
    float* sDG = sm;                   // [64][P]
    float* sRed = sDG + kC * P;        // [16][D] column partial sums of dz
    float* sDb = sRed + 16 * D;        // [64][TC] row partial sums of dbeta
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = rm + 16 * i;
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        const int d = cn + TC * j;
        sDG[c * P + d] = (c < cr.len) ? gG_[in_idx(c, d)] : 0.f;
      }
      sDb[c * TC + cn] = dbr[i];
    }
#pragma unroll
    for (int j = 0; j < NJ; ++j) sRed[rm * D + cn + TC * j] = dzp[j];
    __syncthreads();
    if (t < D) {
      float acc = dgc * ex2(GL[(kC - 1) * D + t]);
      for (int r = 0; r < 16; ++r) acc += sRed[r * D + t];
      for (int c = kC - 1; c >= 0; --c) {
        acc += sDG[c * P + t];
        if (c < cr.len) a.dg[in_idx(c, t)] = acc;
      }
    }
    if (t < kC && t < cr.len) {
      float acc = 0.f;
      for (int j = 0; j < TC; ++j) acc += sDb[t * TC + j];
      a.dbeta[(cr.row0 + t) * H + h] = acc;
    }
  }
}

template <int D, int DTQ, int DTG, int DO>
hipError_t launch_bwd_t(const BwdArgs& a, hipStream_t s) {
  const int chunk_heads = a.B * a.NT * a.H;
  const int chains = a.B * a.H;
  hipLaunchKernelGGL((kda_bwd_prep_kernel<D, DTQ, DTG>), dim3(chunk_heads), dim3(kPrepThreads), 0, s, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int scan_grid = (chains + 7) / 8 * 8 * (D / 32);
  hipLaunchKernelGGL((kda_bwd_fscan_kernel<D>), dim3(scan_grid), dim3(kScanThreads), 0, s, a);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((kda_bwd_rscan_kernel<D, DO>), dim3(scan_grid), dim3(kScanThreads), 0, s, a);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((kda_bwd_chunk_kernel<D, DTQ, DTG, DO>), dim3(chunk_heads), dim3(kChunkThreads), 0, s, a);
  return hipGetLastError();
}

template <int D, int DO>
hipError_t launch_bwd_dt(const BwdArgs& a, int in_dtype, hipStream_t s) {
  switch (in_dtype) {
    case 0: return launch_bwd_t<D, 0, 0, DO>(a, s);
    case 1: return launch_bwd_t<D, 1, 1, DO>(a, s);
    case 2: return launch_bwd_t<D, 2, 2, DO>(a, s);
    default: return launch_bwd_t<D, 1, 0, DO>(a, s);
  }
}

__global__ __launch_bounds__(kThreads) void kda_copy_or_zero_kernel(float* dst, const float* src, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * kThreads)
    dst[i] = (src != nullptr) ? src[i] : 0.f;
}

}  // namespace

hipError_t launch_copy_or_zero(float* dst, const float* src, int64_t n, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  const int64_t blocks = (n + kThreads - 1) / kThreads;
  const int grid = static_cast<int>(blocks < 4096 ? blocks : 4096);
  hipLaunchKernelGGL(kda_copy_or_zero_kernel, dim3(grid), dim3(kThreads), 0, s, dst, src, n);
  return hipGetLastError();
}

hipError_t launch_bwd(const BwdArgs& a, int d, int in_dtype, int do_dtype, hipStream_t s) {
  if (d == 128) return do_dtype == 0 ? launch_bwd_dt<128, 0>(a, in_dtype, s) : launch_bwd_dt<128, 1>(a, in_dtype, s);
  return do_dtype == 0 ? launch_bwd_dt<64, 0>(a, in_dtype, s) : launch_bwd_dt<64, 1>(a, in_dtype, s);
}

}  // namespace kda
