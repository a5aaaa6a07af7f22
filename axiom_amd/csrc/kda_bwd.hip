// Chunked KDA backward (dense [B, T, H, d] inputs).
//
// Gradients of o = chunk_fwd(q, k, v, g, beta, h0) and of the final state
// with respect to q, k, v, g (the log decay), beta and h0, following the
// reference's analytic adjoint per chunk (net/kernels/kda_cc_fused_bwd.py:30-55,
// code :139-228) scanned in reverse over the chunks
// (net/kernels/kda_cc_fused_persist.py:794-842, reference_bwd_scan).  Four
// launches:
//   kda_bwd_prep_kernel   one workgroup per chunk-head: in-chunk log2 cumsum G,
//                         gamma*q, lambda*k, gamma_C, Aqk, T = (I+L)^-1, W, U;
//   forward state scan    one workgroup per (chain, 32 value columns): every
//                         chunk's incoming state S and its v~ = U - W S;
//   reverse scan          same grid, chunks in reverse: the state cotangent
//                         dS entering each chunk from the right, and
//                         dv~ = (lambda k) dS + Aqk^T do;
//                         dS <- gamma_C dS + (gamma q)^T do - W^T dv~; dh0;
//   kda_bwd_chunk_kernel  one workgroup per chunk-head: the rest of the adjoint
//                         (dY, dgq, dW, the two transposed solves, dL, dAqk, the
//                         score adjoints, the cumsum adjoint) and the outputs.
// Two precisions of the workspace, chosen by the input dtype:
//  * fp32 inputs: every workspace array fp32 row-major per chunk-head
//    ch = (b * NT + n) * H + h; scans kda_bwd_fscan_kernel and
//    kda_bwd_rscan_kernel (16 waves, operands split into bf16 hi/lo planes
//    in LDS each chunk step).
//  * 16-bit inputs (bf16, fp16): the forward-side arrays gamma q, lambda k,
//    Aqk, T, W and the stored state S are fp16 (BwdWs<true>: the operand
//    width the forward's own kernels give them), and the
//    prep kernel writes the scans' operands directly as MFMA lane fragments
//    (FL, FA, FQ, FW, FWN, FLT); G, gamma_C, U, v~ and the cotangents dS', dv~
//    stay fp32.  Scans kda_bwd_fscan16_kernel and kda_bwd_rscan16_kernel in
//    the column-owner form: two compute waves (one 16-column tile each of the
//    32-column slice, the state slice in their accumulators) and four
//    producer waves that load two chunks ahead into registers, fill a
//    double-buffered LDS chunk, and store the compute waves' staged outputs
//    a step later; one barrier per chunk step.
// Products: fp16 operands on v_mfma_f32_16x16x32_f16 (exact products of the
// stored values); fp32 operands (cotangents, v~, U, S in the fp32 path) as
// hi/lo pairs of a 16-bit type, about 2^-16 of each product dropped (the
// 16-bit scans scale each column's cotangent by a power of two first, so the
// fp16 pair keeps ~22 bits whatever its range); the rest (prep scores, phase 4
// of the chunk kernel) on v_mfma_f32_16x16x4f32.  Decay factors of
// off-diagonal 16-row tiles are anchored at the row tile's first row
// (2^(G_c - G_a) * 2^(G_a - G_i), both <= 1); diagonal tiles likewise when
// the tile's decay span allows (kDiagAnchorLog2), else per element.
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
// Scan workgroups: one per (chain, 32-column slice).  The scans are bound by
// the latency of their serial chunk steps (operand splits into LDS, three
// barriers and two short MFMA chains per step), so d = 128 runs 16 waves (four
// per SIMD: one state tile and half the operand splitting per wave), d = 64
// eight.
template <int D>
struct ScanThreads {
  static constexpr int value = (D == 128) ? 1024 : 512;
};
constexpr int kScanThreads = 512;   // threads of the 64-column transposed tiles of the scans
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

constexpr int cmax(int a, int b) { return a > b ? a : b; }

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
// Tile::PER pieces of four elements) and the LDS writes.  Split, a scan kernel
// issues the next chunk's loads before the current chunk's arithmetic.
//
// Workspace arrays are fp32 (ET 0) or fp16 (ET 2, see BwdWs); an fp16 tile
// loads 8 bytes per piece and converts when it is written to LDS, so the wait
// for the load falls there, not at the fetch.
template <int ET>
struct WsPiece {
  typedef uint2 t;
};
template <>
struct WsPiece<0> {
  typedef float4 t;
};
template <int ET>
__device__ __forceinline__ float4 ws_unpack(const typename WsPiece<ET>::t& w) {
  if constexpr (ET == 0) {
    return w;
  } else {
    const f4 v = unpack4<ET>(w);
    return make_float4(v[0], v[1], v[2], v[3]);
  }
}
// element `off` of a workspace array of element type ET
template <int ET>
__device__ __forceinline__ const void* ws_at(const float* base, int64_t off) {
  if constexpr (ET == 0) return base + off;
  else return reinterpret_cast<const u16*>(base) + off;
}
template <int ET>
__device__ __forceinline__ void ws_st(float* base, int64_t off, float x) {
  static_assert(ET == 0 || ET == 2, "workspace arrays are fp32 or fp16");
  if constexpr (ET == 0) base[off] = x;
  else reinterpret_cast<u16*>(base)[off] = __builtin_bit_cast(u16, static_cast<_Float16>(x));
}
// four consecutive elements (off a multiple of 4)
template <int ET>
__device__ __forceinline__ void ws_st4(float* base, int64_t off, float4 x) {
  if constexpr (ET == 0) {
    *reinterpret_cast<float4*>(base + off) = x;
  } else {
    static_assert(ET == 2, "workspace arrays are fp32 or fp16");
    typedef _Float16 hv4 __attribute__((ext_vector_type(4)));
    const hv4 v = {static_cast<_Float16>(x.x), static_cast<_Float16>(x.y), static_cast<_Float16>(x.z),
                   static_cast<_Float16>(x.w)};
    *reinterpret_cast<uint2*>(reinterpret_cast<u16*>(base) + off) = __builtin_bit_cast(uint2, v);
  }
}

// four fp32 -> packed fp16 (round to nearest even)
__device__ __forceinline__ uint2 pack_f16x4(const f4& x) {
  const h4 v = {static_cast<_Float16>(x[0]), static_cast<_Float16>(x[1]), static_cast<_Float16>(x[2]),
                static_cast<_Float16>(x[3])};
  return __builtin_bit_cast(uint2, v);
}

// Element types of the backward's workspace.  fp32 inputs keep every array
// fp32.  16-bit inputs store six forward-side arrays in fp16 (gamma q,
// lambda k, Aqk, T, W and the chunk's incoming state S: the operand width the
// forward's own kernels use for them); G, gamma_C, U, v~ (U - W S cancels, so
// their rounding would reach the gradients amplified) and the cotangents dS,
// dv~ (whose scale is the caller's) stay fp32.
template <bool WS16>
struct BwdWs {
  static constexpr int F = WS16 ? 2 : 0;
};

template <int ROWS, int COLS, int NTH = kThreads, int ET = 0>
struct Tile {
  static constexpr int V = COLS / 4;
  static constexpr int N = ROWS * V;
  static constexpr int PER = (N + NTH - 1) / NTH;
  static_assert(COLS % 4 == 0, "four-element pieces");
  typedef typename WsPiece<ET>::t Piece;
  Piece r[PER];
  __device__ __forceinline__ void fetch(const void* src, int src_ld, int col0) {
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int e = threadIdx.x + p * NTH;
      if (N % NTH == 0 || e < N) {
        const int row = e / V, c4 = e - row * V;
        const int64_t i = static_cast<int64_t>(row) * src_ld + col0 + 4 * c4;
        if constexpr (ET == 0) r[p] = *reinterpret_cast<const float4*>(static_cast<const float*>(src) + i);
        else r[p] = *reinterpret_cast<const uint2*>(static_cast<const u16*>(src) + i);
      }
    }
  }
  __device__ __forceinline__ float4 get(int p) const { return ws_unpack<ET>(r[p]); }
  template <int PITCH>
  __device__ __forceinline__ void put(float* dst) const {
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int e = threadIdx.x + p * NTH;
      if (N % NTH == 0 || e < N) {
        const int row = e / V, c4 = e - row * V;
        const float4 x = get(p);
        float* d = dst + row * PITCH + 4 * c4;
        d[0] = x.x;
        d[1] = x.y;
        d[2] = x.z;
        d[3] = x.w;
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

// Largest in-tile decay (log2 units, one channel) at which the chunk
// kernel's diagonal score-adjoint tiles run on the matrix cores anchored at
// the tile's first row: the key factors reach 2^kDiagAnchorLog2, which leaves
// 2^96 of fp32's range for the cotangent sums they multiply.
constexpr float kDiagAnchorLog2 = 32.f;

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
  // every thread loads (masked ones from row 0 of the chunk) and zeroes
  // where it stores, so no load sits inside a branch
  float tmp[PER][8];
#pragma unroll
  for (int p = 0; p < PER; ++p) {
    const int e = threadIdx.x + p * NTH;
    const int r = e / V, c8 = e - r * V;
    const bool ok = (N % NTH == 0 || e < N) && r < len;
    ld8<DT>(src, ((row0 + (ok ? r : 0)) * H + h) * D + col0 + 8 * (ok ? c8 : 0), tmp[p]);
  }
#pragma unroll
  for (int p = 0; p < PER; ++p) {
    const int e = threadIdx.x + p * NTH;
    if (N % NTH == 0 || e < N) {
      const int r = e / V, c8 = e - r * V;
      const bool ok = r < len;
#pragma unroll
      for (int x = 0; x < 8; ++x) dst[r * PITCH + 8 * c8 + x] = ok ? tmp[p][x] * mul : 0.f;
    }
  }
}

// lds_load_in split into its loads (fetch) and its LDS writes (put), so a
// kernel can issue the loads of a later phase before this phase's arithmetic.
template <int DT, int D, int COLS, int NTH>
struct InTile {
  static constexpr int V = COLS / 8;
  static constexpr int N = kC * V;
  static constexpr int PER = (N + NTH - 1) / NTH;
  static_assert(COLS % 8 == 0, "8-element loads");
  uint4 w[DT == 0 ? 2 * PER : PER];
  __device__ __forceinline__ void fetch(const void* src, int64_t row0, int len, int H, int h, int col0) {
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int e = threadIdx.x + p * NTH;
      const int r = e / V, c8 = e - r * V;
      const bool ok = (N % NTH == 0 || e < N) && r < len;
      const int64_t i = ((row0 + (ok ? r : 0)) * H + h) * D + col0 + 8 * c8;
      // the address is valid for every thread (row 0 when masked): load
      // unconditionally, then zero, so no load sits inside a branch
      const uint4 z = make_uint4(0, 0, 0, 0);
      if constexpr (DT == 0) {
        const uint4* q = reinterpret_cast<const uint4*>(static_cast<const float*>(src) + i);
        const uint4 v0 = q[0], v1 = q[1];
        w[2 * p] = ok ? v0 : z;
        w[2 * p + 1] = ok ? v1 : z;
      } else {
        const uint4 v = *reinterpret_cast<const uint4*>(static_cast<const u16*>(src) + i);
        w[p] = ok ? v : z;
      }
    }
  }
  template <int PITCH>
  __device__ __forceinline__ void put(float* dst, float mul) const {
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int e = threadIdx.x + p * NTH;
      if (N % NTH == 0 || e < N) {
        const int r = e / V, c8 = e - r * V;
        float x[8];
        if constexpr (DT == 0) {
          const uint4 a = w[2 * p], b = w[2 * p + 1];
          x[0] = __uint_as_float(a.x); x[1] = __uint_as_float(a.y); x[2] = __uint_as_float(a.z); x[3] = __uint_as_float(a.w);
          x[4] = __uint_as_float(b.x); x[5] = __uint_as_float(b.y); x[6] = __uint_as_float(b.z); x[7] = __uint_as_float(b.w);
        } else {
          const f4 lo = unpack4<DT>(make_uint2(w[p].x, w[p].y)), hi = unpack4<DT>(make_uint2(w[p].z, w[p].w));
#pragma unroll
          for (int q = 0; q < 4; ++q) { x[q] = lo[q]; x[4 + q] = hi[q]; }
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) dst[r * PITCH + 8 * c8 + q] = x[q] * mul;
      }
    }
  }
};

// ---------------------------------------------------------------------------
// prep: G, gamma*q, lambda*k, gamma_C, Aqk, T, W, U of one chunk-head
// ---------------------------------------------------------------------------
__device__ __forceinline__ f4 mfma4(float a, float b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Index of the stored Aqk^T A fragment (key tile it, K step kb over the query
// rows): (0,0) (0,1) (1,0) (1,1) (2,1) (3,1); (2,0) and (3,0) are zero and
// not stored.
__device__ __forceinline__ int fa_frag(int it, int kb) { return (it < 2) ? 2 * it + kb : it + 2; }

// The chunk's channels are taken in halves of 64 (d = 128) so the shared
// memory fits two workgroups per CU: the scores accumulate over the halves in
// registers, T = (I+L)^-1 is built once, and W, U are formed per half of
// their columns (the last half's k and G still staged, the other reloaded).
template <int D, int DTQ, int DTG>
__global__ __launch_bounds__(kPrepThreads, 4) void kda_bwd_prep_kernel(BwdArgs a) {
  constexpr int EF = BwdWs<DTQ != 0>::F;   // gamma q, lambda k, Aqk, T, W, U
  constexpr int HD = 64;              // channels per half
  constexpr int NHALF = D / HD;
  // [64][HD] pitch: row fragments conflict-free (rows 4 banks apart), rows
  // 16-byte aligned for the diagonal tiles' vector reads
  constexpr int P = HD + 4;
  constexpr int PC = kC + 1;
  static_assert(kC * PC <= kC * P, "T shares sQ's buffer");
  __shared__ __attribute__((aligned(16))) float sQ[kC * P], sK[kC * P], sG[kC * P];   // one channel half; sQ then holds T
  __shared__ float sL[kC * PC];       // L, then one half of beta*v
  __shared__ float sTmp[768];         // the triangular inversion's scratch
  __shared__ float sB[kC];
  constexpr int NTH = kPrepThreads;
  const int t = threadIdx.x;
  const int wv = t >> 6, l = t & 63, r16 = l & 15, gq = l >> 4;
  const int H = a.H;
  const int u = blockIdx.x / H, h = blockIdx.x - u * H;
  const ChunkRows cr = chunk_rows(a, u);
  const int64_t ch = static_cast<int64_t>(u) * H + h;
  float* const sT = sQ;

  // k and the in-chunk inclusive cumsum of g (log2 units) of channel half c0
  // (both tiles' loads issued before either is stored)
  auto stage_k_g = [&](int c0) {
    InTile<DTQ, D, HD, NTH> ik;
    InTile<DTG, D, HD, NTH> ig;
    ik.fetch(a.k, cr.row0, cr.len, H, h, c0);
    ig.fetch(a.g, cr.row0, cr.len, H, h, c0);
    ik.template put<P>(sK, 1.f);
    ig.template put<P>(sG, 1.f);
  };
  // every thread: channel t % HD, rows 8 s .. 8 s + 7 (s = t / HD): the
  // prefix over its rows, then the sums of the segments above it (through
  // sTmp, which the triangular inversion alone uses otherwise); ends with a
  // barrier before which sG must not be read
  static_assert(NTH == 8 * HD && kC == 64, "eight 8-row segments per channel");
  auto cumsum_g = [&]() {
    const int d = t & (HD - 1), s8 = t / HD;
    float x[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) x[j] = sG[(8 * s8 + j) * P + d];
#pragma unroll
    for (int j = 1; j < 8; ++j) x[j] += x[j - 1];
    sTmp[s8 * HD + d] = x[7];
    __syncthreads();
    float pre = 0.f;
    for (int k = 0; k < s8; ++k) pre += sTmp[k * HD + d];
#pragma unroll
    for (int j = 0; j < 8; ++j) sG[(8 * s8 + j) * P + d] = (x[j] + pre) * kLog2e;
  };

  // scores: Aqk (c >= i) to the workspace, L = beta_c Akk (c > i) to LDS,
  // accumulated over the channel halves on the matrix cores, one 16 x 16 tile
  // pair per wave: waves 0..5 the off-diagonal pairs (row tile R > key tile
  // s), waves 6 and 7 two diagonal tiles each.  The decay is factored at the
  // row tile's first row a, 2^(G_c - G_i) = 2^(G_c - G_a) 2^(G_a - G_i), and
  // applied to each operand element as it is read: both factors <= 1 off the
  // diagonal; on it the key factor is >= 1, up to the tile's decay, and pairs
  // where the product would exceed 1 are masked.  A diagonal tile that decays
  // by more than 2^-kDiagAnchorLog2 in a channel of the half takes
  // 2^(G_c - G_i) per element for that half instead (lane (r, gq) forming its
  // own four outputs, rows 4 gq + e, key r).
  const int R_off = (wv < 1) ? 1 : (wv < 3) ? 2 : 3;
  const int sk_off = wv - R_off * (R_off - 1) / 2;
  const int NPAIR = (wv < 6) ? 1 : 2;   // wave-uniform
  auto pair_rs = [&](int pi, int& R, int& sk) {
    if (wv < 6) { R = R_off; sk = sk_off; }
    else { R = 2 * (wv - 6) + pi; sk = R; }
  };
  f4 accA[2], accL[2];
#pragma unroll
  for (int pi = 0; pi < 2; ++pi) accA[pi] = accL[pi] = f4{0.f, 0.f, 0.f, 0.f};
  // the next half's q, k, g and beta, loaded during this half's scores
  InTile<DTQ, D, HD, NTH> nq, nk;
  InTile<DTG, D, HD, NTH> ng;
  float nb = 0.f;
  auto fetch_half = [&](int c0) {
    nq.fetch(a.q, cr.row0, cr.len, H, h, c0);
    nk.fetch(a.k, cr.row0, cr.len, H, h, c0);
    ng.fetch(a.g, cr.row0, cr.len, H, h, c0);
    const int tb = t & (kC - 1);
    nb = ld1<DTG>(a.beta, (cr.row0 + (tb < cr.len ? tb : 0)) * H + h);
  };
  fetch_half(0);
  for (int hf = 0; hf < NHALF; ++hf) {
    const int c0 = HD * hf;
    if (hf > 0) __syncthreads();      // the previous half's reads are done
    nq.template put<P>(sQ, a.scale);
    nk.template put<P>(sK, 1.f);
    ng.template put<P>(sG, 1.f);
    if (hf == 0 && t < kC) sB[t] = (t < cr.len) ? nb : 0.f;
    __syncthreads();
    cumsum_g();
    __syncthreads();
    {
      if constexpr (EF == 0) {
        // gamma q and lambda k, row-major
        const int64_t base = ch * kC * D + c0;
        constexpr int V4 = HD / 4;      // float4 groups per row
        for (int e = t; e < kC * V4; e += NTH) {
          const int c = e / V4, d = 4 * (e - c * V4);
          const float4 gl = *reinterpret_cast<const float4*>(&sG[c * P + d]);
          const float4 gz = *reinterpret_cast<const float4*>(&sG[(kC - 1) * P + d]);
          const float4 qv = *reinterpret_cast<const float4*>(&sQ[c * P + d]);
          const float4 kv = *reinterpret_cast<const float4*>(&sK[c * P + d]);
          const float4 qg = make_float4(ex2(gl.x) * qv.x, ex2(gl.y) * qv.y, ex2(gl.z) * qv.z, ex2(gl.w) * qv.w);
          const float4 kl = make_float4(ex2(gz.x - gl.x) * kv.x, ex2(gz.y - gl.y) * kv.y, ex2(gz.z - gl.z) * kv.z,
                                        ex2(gz.w - gl.w) * kv.w);
          ws_st4<EF>(a.QG, base + c * D + d, qg);
          ws_st4<EF>(a.KL, base + c * D + d, kl);
        }
      } else {
        // the reverse scan's A fragments of this half's channels, one lane
        // fragment per thread each (the slot order of kda_internal.h)
        static_assert(NTH == 512 && HD == 64, "one (gamma q)^T and one lambda k lane fragment per thread");
        const int ln = t & 63, rr = ln & 15, g4 = ln >> 4, hi = (t >> 6) & 1, tt = t >> 7;
        h8 vq, vl, vt;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          // (gamma q)^T and (lambda k)^T: channel tile tt of the half, K step hi over the rows
          const int c = 32 * hi + 4 * g4 + (e & 3) + 16 * (e >> 2), dq = 16 * tt + rr;
          vq[e] = static_cast<_Float16>(ex2(sG[c * P + dq]) * sQ[c * P + dq]);
          vt[e] = static_cast<_Float16>(ex2(sG[(kC - 1) * P + dq] - sG[c * P + dq]) * sK[c * P + dq]);
          // lambda k: row tile tt, K step hi over the half's channels
          const int row = 16 * tt + rr, dl = 32 * hi + 4 * g4 + (e & 3) + 16 * (e >> 2);
          vl[e] = static_cast<_Float16>(ex2(sG[(kC - 1) * P + dl] - sG[row * P + dl]) * sK[row * P + dl]);
        }
        const int dt = (c0 >> 4) + tt, j = (c0 >> 5) + hi;
        *reinterpret_cast<h8*>(static_cast<_Float16*>(a.FQ) + (((ch * (D / 16) + dt) * 2 + hi) * 64 + ln) * 8) = vq;
        *reinterpret_cast<h8*>(static_cast<_Float16*>(a.FLT) + (((ch * (D / 16) + dt) * 2 + hi) * 64 + ln) * 8) = vt;
        *reinterpret_cast<h8*>(static_cast<_Float16*>(a.FL) + (((ch * 4 + tt) * (D / 32) + j) * 64 + ln) * 8) = vl;
      }
      if (t < HD) a.GCV[ch * D + c0 + t] = ex2(sG[(kC - 1) * P + t]);
    }
    if (hf + 1 < NHALF) fetch_half(c0 + HD);
#pragma unroll
    for (int pi = 0; pi < 2; ++pi) {
      if (pi >= NPAIR) break;
      int R, sk;
      pair_rs(pi, R, sk);
      const int a0 = 16 * R, i = 16 * sk + r16;
      // a diagonal tile decaying past the anchor's range in a channel of the half
      bool far = false;
      if (R == sk) {
#pragma unroll
        for (int k = 0; k < HD / 4; ++k) {
          const int d = 4 * k + gq;
          far |= sG[a0 * P + d] - sG[(a0 + 15) * P + d] > kDiagAnchorLog2;
        }
      }
      if (!__any(far)) {
#pragma unroll 8
        for (int k = 0; k < HD / 4; ++k) {
          const int d = 4 * k + gq;
          const float ga = sG[a0 * P + d];
          const float fa = ex2(sG[(a0 + r16) * P + d] - ga);
          const float bk = sK[i * P + d] * ex2(ga - sG[i * P + d]);
          accA[pi] = mfma4(sQ[(a0 + r16) * P + d] * fa, bk, accA[pi]);
          accL[pi] = mfma4(sK[(a0 + r16) * P + d] * fa, bk, accL[pi]);
        }
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int c = a0 + 4 * gq + e;
          if (r16 > 4 * gq + e) continue;   // above the diagonal (masked below)
          float sA = 0.f, sL4 = 0.f;
#pragma unroll 2
          for (int d4 = 0; d4 < HD; d4 += 4) {
            const float4 kI = *reinterpret_cast<const float4*>(&sK[i * P + d4]);
            const float4 gI = *reinterpret_cast<const float4*>(&sG[i * P + d4]);
            const float4 gC = *reinterpret_cast<const float4*>(&sG[c * P + d4]);
            const float4 qC = *reinterpret_cast<const float4*>(&sQ[c * P + d4]);
            const float4 kC4 = *reinterpret_cast<const float4*>(&sK[c * P + d4]);
            const float ki[4] = {kI.x * ex2(gC.x - gI.x), kI.y * ex2(gC.y - gI.y), kI.z * ex2(gC.z - gI.z),
                                 kI.w * ex2(gC.w - gI.w)};
            const float qc[4] = {qC.x, qC.y, qC.z, qC.w}, kc[4] = {kC4.x, kC4.y, kC4.z, kC4.w};
#pragma unroll
            for (int x = 0; x < 4; ++x) {
              sA = fmaf(qc[x], ki[x], sA);
              sL4 = fmaf(kc[x], ki[x], sL4);
            }
          }
          accA[pi][e] += sA;
          accL[pi][e] += sL4;
        }
      }
    }
  }
  const int64_t aq0 = ch * kC * kC;
#pragma unroll
  for (int pi = 0; pi < 2; ++pi) {
    if (pi >= NPAIR) break;
    int R, sk;
    pair_rs(pi, R, sk);
    const int a0 = 16 * R, i = 16 * sk + r16;
    f4 vA;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int c = a0 + 4 * gq + e;
      const bool diag = R == sk;
      vA[e] = (!diag || r16 <= 4 * gq + e) ? accA[pi][e] : 0.f;   // Aqk: i <= c
      if constexpr (EF == 0) ws_st<EF>(a.AQ, aq0 + c * kC + i, vA[e]);
      sL[c * PC + i] = (!diag || r16 < 4 * gq + e) ? accL[pi][e] * sB[c] : 0.f;   // L: i < c
    }
    if constexpr (EF != 0)   // Aqk^T fragment (key tile sk, K step R / 2), half R % 2
      *reinterpret_cast<uint2*>(static_cast<u16*>(a.FA) + ((ch * 6 + fa_frag(sk, R >> 1)) * 64 + l) * 8 +
                                4 * (R & 1)) = pack_f16x4(vA);
  }
  // blocks above the diagonal: zero
  for (int e = t; e < 6 * 256; e += NTH) {
    const int blk = e >> 8, rc = (e >> 4) & 15, ri = e & 15;
    const int R = (blk < 3) ? 0 : (blk < 5) ? 1 : 2;             // (0,1) (0,2) (0,3) (1,2) (1,3) (2,3)
    const int sk = (blk < 3) ? blk + 1 : (blk < 5) ? blk - 1 : 3;
    const int c = 16 * R + rc, i = 16 * sk + ri;
    if constexpr (EF == 0) ws_st<EF>(a.AQ, aq0 + c * kC + i, 0.f);
    sL[c * PC + i] = 0.f;
  }
  if constexpr (EF != 0) {
    // the zero halves of the stored Aqk^T fragments: key tile 1 against row
    // tile 0, key tile 3 against row tile 2
    if (t < 128)
      *reinterpret_cast<uint2*>(static_cast<u16*>(a.FA) +
                                ((ch * 6 + (t < 64 ? fa_frag(1, 0) : fa_frag(3, 1))) * 64 + (t & 63)) * 8) =
          uint2{0u, 0u};
  }
  __syncthreads();

  // T = (I + L)^-1 (into sQ's buffer: q is no longer read); the first W/U
  // pass's v half is loaded during the inversion
  InTile<DTQ, D, HD, NTH> iv;
  iv.fetch(a.v, cr.row0, cr.len, H, h, HD * (NHALF - 1));
  invert_unit_lower64<PC, NTH>(sL, sT, sTmp);
  {
    static_assert(kC * kC == 8 * NTH, "eight entries of T per thread");
    const int c = t >> 3, i0 = 8 * (t & 7);
    const float* row = sT + c * PC + i0;
    const int64_t o = ch * kC * kC + c * kC + i0;
    ws_st4<EF>(a.TM, o, make_float4(row[0], row[1], row[2], row[3]));
    ws_st4<EF>(a.TM, o + 4, make_float4(row[4], row[5], row[6], row[7]));
  }
  // W = T (beta gamma k), U = T (beta v) on the matrix cores, per half of
  // their columns (the last half first: its k and G are still staged); wave
  // wv owns row tile wv / 2 and column tiles (wv % 2) HD/32 + q of the half
  float* const sV = sL;               // beta * v of the half, pitch PC
  for (int pass = 0; pass < NHALF; ++pass) {
    const int c0 = HD * (NHALF - 1 - pass);
    if (pass > 0) {
      __syncthreads();                // the previous pass's products are done
      iv.fetch(a.v, cr.row0, cr.len, H, h, c0);   // in flight during the k, g staging
      stage_k_g(c0);
      __syncthreads();
      cumsum_g();
    }
    iv.template put<PC>(sV, 1.f);
    __syncthreads();
    for (int e = t; e < kC * HD; e += NTH) {
      const int c = e / HD, d = e - c * HD;
      sK[c * P + d] *= sB[c] * ex2(sG[c * P + d]);
      sV[c * PC + d] *= sB[c];
    }
    __syncthreads();
    constexpr int NDT = HD / 32;
    const int mt = wv >> 1, dg = wv & 1;
    const int mts = __builtin_amdgcn_readfirstlane(mt);
    f4 accW[NDT], accU[NDT];
#pragma unroll
    for (int q = 0; q < NDT; ++q)
#pragma unroll
      for (int e = 0; e < 4; ++e) accW[q][e] = accU[q][e] = 0.f;
    // T[c][i] is zero for i > c: row tile mt needs K steps i < 16 (mt + 1) only
#pragma unroll 4
    for (int k = 0; k < 4 * (mts + 1); ++k) {
      const float at = sT[(16 * mt + r16) * PC + 4 * k + gq];
#pragma unroll
      for (int q = 0; q < NDT; ++q) {
        const int col = 16 * (dg * NDT + q) + r16;
        accW[q] = mfma4(at, sK[(4 * k + gq) * P + col], accW[q]);
        accU[q] = mfma4(at, sV[(4 * k + gq) * PC + col], accU[q]);
      }
    }
    const int64_t wu0 = ch * kC * D + c0;
#pragma unroll
    for (int q = 0; q < NDT; ++q)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int o = (16 * mt + 4 * gq + e) * D + 16 * (dg * NDT + q) + r16;
        if constexpr (EF == 0) ws_st<EF>(a.WM, wu0 + o, accW[q][e]);
        a.UM[wu0 + o] = accU[q][e];
      }
    if constexpr (EF != 0) {
      // W^T fragments: channel tile of column tile q, K step mt / 2, half mt % 2;
      // W fragments (rows x channels) of K step c0 / 32 + dg: the D-layout tile
      // read as an A fragment is W^T, and its product with the identity lands
      // row r of W, channels 4 gq .. 4 gq + 3 of the tile, in lane (r, gq)
      static_assert(NDT == 2, "two column tiles per wave: one 32-channel K step");
      h4 ident;
#pragma unroll
      for (int i = 0; i < 4; ++i) ident[i] = static_cast<_Float16>((4 * gq + i == r16) ? 1.f : 0.f);
      h8 wn;
#pragma unroll
      for (int q = 0; q < NDT; ++q) {
        const int dt = (c0 >> 4) + dg * NDT + q;
        const uint2 w16 = pack_f16x4(accW[q]);
        *reinterpret_cast<uint2*>(static_cast<u16*>(a.FW) + (((ch * (D / 16) + dt) * 2 + (mt >> 1)) * 64 + l) * 8 +
                                  4 * (mt & 1)) = w16;
        const f4 tr = mma16(f4{0.f, 0.f, 0.f, 0.f}, __builtin_bit_cast(h4, w16), ident);
#pragma unroll
        for (int i = 0; i < 4; ++i) wn[4 * q + i] = static_cast<_Float16>(tr[i]);
      }
      *reinterpret_cast<h8*>(static_cast<_Float16*>(a.FWN) + (((ch * 4 + mt) * (D / 32) + (c0 >> 5) + dg) * 64 + l) * 8) = wn;
    }
  }
}

// ---------------------------------------------------------------------------
// The scans run their products on the bf16 matrix cores as hi/lo triples
// (v_mfma_f32_16x16x32_bf16): lane (r = l & 15, gq = l >> 4) supplies
// A[r][32 s + 8 gq .. + 7] and B[32 s + 8 gq .. + 7][r] of K block s and
// holds D rows 4 gq + i, column r.  Eight waves per workgroup; the 32-column
// state slice is (D/16) x 2 tiles in accumulators, D/64 tiles per wave; the
// [64][32] results of a chunk are 8 tiles, one per wave.  Operands sit in LDS
// as hi and lo bf16 planes with the K index contiguous, so each fragment is
// one 16-byte read.
// ---------------------------------------------------------------------------
constexpr int kPB = 48;   // fp32 pitch of the forward scan's [64][32] U slice

// x0, x1 -> packed bf16 pairs hi (round to nearest even) and lo = bf16(x - hi)
__device__ __forceinline__ void split2_bf16(float x0, float x1, unsigned& h, unsigned& l) {
  h = pack_bf16x2(x0, x1);
  l = pack_bf16x2(x0 - __uint_as_float(h << 16), x1 - __uint_as_float(h & 0xFFFF0000u));
}
// hi * hi + hi * lo + lo * hi of one 32-wide K block on the bf16 matrix cores
// (products exact, sums fp32; the dropped lo * lo term and the rounding of lo
// leave about 2^-16 of each product)
__device__ __forceinline__ f4 mma3_bf16(f4 acc, const b8& ah, const b8& al, const b8& bh, const b8& bl) {
  acc = mma32_bf16(acc, ah, bh);
  acc = mma32_bf16(acc, ah, bl);
  return mma32_bf16(acc, al, bh);
}

// A fetched fp32 tile into LDS as hi / lo bf16 planes (row pitch PB bf16).
template <int PB, int ROWS, int COLS, int NTH, int ET>
__device__ __forceinline__ void put_hl(const Tile<ROWS, COLS, NTH, ET>& tl, __bf16* h, __bf16* l) {
  typedef Tile<ROWS, COLS, NTH, ET> TT;
#pragma unroll
  for (int p = 0; p < TT::PER; ++p) {
    const int e = threadIdx.x + p * NTH;
    if (TT::N % NTH == 0 || e < TT::N) {
      const int row = e / TT::V, c4 = e - row * TT::V;
      const float4 x = tl.get(p);
      uint2 hh, ll;
      split2_bf16(x.x, x.y, hh.x, ll.x);
      split2_bf16(x.z, x.w, hh.y, ll.y);
      *reinterpret_cast<uint2*>(&h[row * PB + 4 * c4]) = hh;
      *reinterpret_cast<uint2*>(&l[row * PB + 4 * c4]) = ll;
    }
  }
}
template <int PB, int DT, int D, int COLS, int NTH>
__device__ __forceinline__ void put_hl(const InTile<DT, D, COLS, NTH>& tl, __bf16* h, __bf16* l) {
  typedef InTile<DT, D, COLS, NTH> TT;
#pragma unroll
  for (int p = 0; p < TT::PER; ++p) {
    const int e = threadIdx.x + p * NTH;
    if (TT::N % NTH == 0 || e < TT::N) {
      const int r = e / TT::V, c8 = e - r * TT::V;
      float x[8];
      if constexpr (DT == 0) {
        const uint4 a = tl.w[2 * p], b = tl.w[2 * p + 1];
        x[0] = __uint_as_float(a.x); x[1] = __uint_as_float(a.y); x[2] = __uint_as_float(a.z); x[3] = __uint_as_float(a.w);
        x[4] = __uint_as_float(b.x); x[5] = __uint_as_float(b.y); x[6] = __uint_as_float(b.z); x[7] = __uint_as_float(b.w);
      } else {
        const f4 lo = unpack4<DT>(make_uint2(tl.w[p].x, tl.w[p].y)), hi = unpack4<DT>(make_uint2(tl.w[p].z, tl.w[p].w));
#pragma unroll
        for (int q = 0; q < 4; ++q) { x[q] = lo[q]; x[4 + q] = hi[q]; }
      }
      uint4 hh, ll;
      split2_bf16(x[0], x[1], hh.x, ll.x);
      split2_bf16(x[2], x[3], hh.y, ll.y);
      split2_bf16(x[4], x[5], hh.z, ll.z);
      split2_bf16(x[6], x[7], hh.w, ll.w);
      *reinterpret_cast<uint4*>(&h[r * PB + 8 * c8]) = hh;
      *reinterpret_cast<uint4*>(&l[r * PB + 8 * c8]) = ll;
    }
  }
}

// A [64][COLS] tile (element type ET) fetched for a transposed store into
// hi / lo bf16 planes [COLS][64] (the source row index becomes the contiguous
// K index): thread t holds rows 2 rp and 2 rp + 1 (rp = t % 32) of the
// four-column groups t / 32 + (NTH / 32) j, so each transposed row is written
// as packed row pairs, consecutive lanes at consecutive words.
template <int COLS, int NTH, int ET = 0>
struct TTile {
  static constexpr int G = NTH / 32;
  static constexpr int PER = (COLS / 4) / G;
  static_assert(NTH % 32 == 0 && (COLS / 4) % G == 0, "transposed tile mapping");
  typedef typename WsPiece<ET>::t Piece;
  Piece r[PER][2];
  __device__ __forceinline__ void fetch(const void* src, int src_ld, int col0) {
#pragma unroll
    for (int j = 0; j < PER; ++j) fetch_block(src, src_ld, col0, j);
  }
  // column block j alone: columns col0 + 4 (cg + G j) .. + 3 of the row pair
  __device__ __forceinline__ void fetch_block(const void* src, int src_ld, int col0, int j) {
    const int rp = threadIdx.x & 31, cg = threadIdx.x >> 5;
#pragma unroll
    for (int y = 0; y < 2; ++y) {
      const int64_t i = static_cast<int64_t>(2 * rp + y) * src_ld + col0 + 4 * (cg + G * j);
      if constexpr (ET == 0) r[j][y] = *reinterpret_cast<const float4*>(static_cast<const float*>(src) + i);
      else r[j][y] = *reinterpret_cast<const uint2*>(static_cast<const u16*>(src) + i);
    }
  }
  // block j row-major into hi / lo planes of pitch PB, block-local columns
  // 4 cg .. 4 cg + 3 (a [rows][4 G] pass of a product over the columns)
  template <int PB>
  __device__ __forceinline__ void put_rows_hl(int j, __bf16* h, __bf16* l) const {
    const int rp = threadIdx.x & 31, cg = threadIdx.x >> 5;
#pragma unroll
    for (int y = 0; y < 2; ++y) {
      const float4 x = ws_unpack<ET>(r[j][y]);
      uint2 hh, ll;
      split2_bf16(x.x, x.y, hh.x, ll.x);
      split2_bf16(x.z, x.w, hh.y, ll.y);
      *reinterpret_cast<uint2*>(&h[(2 * rp + y) * PB + 4 * cg]) = hh;
      *reinterpret_cast<uint2*>(&l[(2 * rp + y) * PB + 4 * cg]) = ll;
    }
  }
  template <int PB>
  __device__ __forceinline__ void put_hl(__bf16* h, __bf16* l) const {
    const int rp = threadIdx.x & 31, cg = threadIdx.x >> 5;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int c4 = 4 * (cg + G * j);
      const float4 y0 = ws_unpack<ET>(r[j][0]), y1 = ws_unpack<ET>(r[j][1]);
      const float x0[4] = {y0.x, y0.y, y0.z, y0.w};
      const float x1[4] = {y1.x, y1.y, y1.z, y1.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        unsigned hh, ll;
        split2_bf16(x0[e], x1[e], hh, ll);
        *reinterpret_cast<unsigned*>(&h[(c4 + e) * PB + 2 * rp]) = hh;
        *reinterpret_cast<unsigned*>(&l[(c4 + e) * PB + 2 * rp]) = ll;
      }
    }
  }
};

// forward state scan of one (chain, 32-column slice): S_in and v~ per chunk.
// The products run as bf16 hi/lo triples (v_mfma_f32_16x16x32_bf16, lane
// (r, gq) holding K values 8 gq .. 8 gq + 7 of each 32-wide block): W and
// (lambda k)^T, the state slice S^T and v~^T are kept in LDS as hi and lo
// bf16 planes with the K index contiguous, so each fragment is one 16-byte
// read.  The state itself stays fp32 in the accumulators.  With 16-bit inputs
// every operand of both products is forward-side and fp16 (W and lambda k as
// stored; S rounded as it is stored, v~ rounded for the product and stored
// in fp32), so each product is one fp16 MFMA per K block, the forward
// kernels' operand precision.
template <int D, bool WS16>
__global__ __launch_bounds__(ScanThreads<D>::value) void kda_bwd_fscan_kernel(BwdArgs a) {
  constexpr int EF = BwdWs<WS16>::F;   // W, lambda k in; S_in out
  constexpr int NTH = ScanThreads<D>::value;
  constexpr int NS = D / 32;
  constexpr int NST = (D / 8) / (NTH / 64);   // state tiles per wave (D / 8 tiles of the 32-column slice)
  static_assert(NST >= 1, "at least one state tile per wave");
  constexpr int PW = D + 8;     // bf16 pitch of rows whose K index is a channel
  constexpr int PK = kC + 8;    // bf16 pitch of rows whose K index is a chunk row
  __shared__ __attribute__((aligned(16))) __bf16 sWh[kC * PW], sWl[kC * PW];    // W [64][D]
  __shared__ __attribute__((aligned(16))) __bf16 sKh[D * PK], sKl[D * PK];      // (lambda k)^T [D][64]
  __shared__ __attribute__((aligned(16))) __bf16 sSh[32 * PW], sSl[32 * PW];    // S^T [32][D]
  __shared__ __attribute__((aligned(16))) __bf16 sVh[32 * PK], sVl[32 * PK];    // v~^T [32][64]
  __shared__ float sU[kC * kPB], sGC[D];
  const int t = threadIdx.x, wv = t >> 6, l = t & 63, r = l & 15, gq = l >> 4;
  const int H = a.H;
  int chain, split;
  if (!scan_slot<NS>(a.B * H, chain, split)) return;   // uniform per workgroup
  const int b = chain / H, h = chain - b * H;
  const int c0 = 32 * split;
  const int mt = wv >> 1, ct = wv & 1;                  // this wave's v~ tile (waves 0-7: 8 tiles)
  const bool vt_wave = wv < 8;
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
  typedef Tile<kC, D, NTH, EF> TD;
  TD tW;
  Tile<kC, 32, NTH> tU;
  // lambda*k, fetched for its transposed store: thread t holds rows 2 rp and
  // 2 rp + 1 (rp = t % 32) of the column groups KCG j + t / 32, so each
  // transposed row is written as packed row pairs, consecutive lanes at
  // consecutive words
  constexpr int KCG = NTH / 32;                    // column groups per pass
  constexpr int KPER = (D / 4) / KCG;              // float4 column groups per thread
  static_assert((D / 4) % KCG == 0, "lambda*k column groups");
  typename WsPiece<EF>::t kq[KPER][2];
  const int rp = t & 31, cg = t >> 5;
  float pgc;   // gamma_C of the chunk, loaded with its operands (every thread; t < D stores it)
  auto fetch = [&](int n) {
    const int64_t ch = (static_cast<int64_t>(b) * a.NT + n) * H + h;
    pgc = a.GCV[ch * D + (t & (D - 1))];
    tW.fetch(ws_at<EF>(a.WM, ch * kC * D), D, 0);
    const void* KLp = ws_at<EF>(a.KL, ch * kC * D);
#pragma unroll
    for (int j = 0; j < KPER; ++j)
#pragma unroll
      for (int y = 0; y < 2; ++y) {
        const int i = (2 * rp + y) * D + 4 * (cg + KCG * j);
        if constexpr (EF == 0) kq[j][y] = *reinterpret_cast<const float4*>(static_cast<const float*>(KLp) + i);
        else kq[j][y] = *reinterpret_cast<const uint2*>(static_cast<const u16*>(KLp) + i);
      }
    tU.fetch(a.UM + ch * kC * D, D, c0);
  };
  if (a.NT > 0) fetch(0);
  for (int n = 0; n < a.NT; ++n) {
    const int64_t ch = (static_cast<int64_t>(b) * a.NT + n) * H + h;
#pragma unroll
    for (int q = 0; q < NST; ++q) {
      const int m0 = 16 * rt[q] + 4 * gq, col = 16 * cs[q] + r;
#pragma unroll
      for (int i = 0; i < 4; ++i) ws_st<EF>(a.SI, ch * D * D + (m0 + i) * D + c0 + col, S[q][i]);
      if constexpr (WS16) {
        *reinterpret_cast<uint2*>(&sSh[col * PW + m0]) = pack_f16x4(S[q]);
      } else {
        uint2 hh, ll;
        split2_bf16(S[q][0], S[q][1], hh.x, ll.x);
        split2_bf16(S[q][2], S[q][3], hh.y, ll.y);
        *reinterpret_cast<uint2*>(&sSh[col * PW + m0]) = hh;
        *reinterpret_cast<uint2*>(&sSl[col * PW + m0]) = ll;
      }
    }
    // W row-major and lambda*k transposed, as hi / lo planes (16-bit
    // workspace: one fp16 plane each, the stored values as they are)
#pragma unroll
    for (int p = 0; p < TD::PER; ++p) {
      const int e = t + p * NTH;
      const int row = e / TD::V, c4 = e - row * TD::V;
      if constexpr (WS16) {
        *reinterpret_cast<uint2*>(&sWh[row * PW + 4 * c4]) = tW.r[p];
      } else {
        const float4 w = tW.get(p);
        uint2 hh, ll;
        split2_bf16(w.x, w.y, hh.x, ll.x);
        split2_bf16(w.z, w.w, hh.y, ll.y);
        *reinterpret_cast<uint2*>(&sWh[row * PW + 4 * c4]) = hh;
        *reinterpret_cast<uint2*>(&sWl[row * PW + 4 * c4]) = ll;
      }
    }
#pragma unroll
    for (int j = 0; j < KPER; ++j) {
      const int ch4 = 4 * (cg + KCG * j);
      if constexpr (WS16) {
        // channel ch4 + e of rows 2 rp, 2 rp + 1: the e-th halves of the two
        // rows' pieces, packed low / high
        const uint2 w0 = kq[j][0], w1 = kq[j][1];
        const unsigned pr[4] = {(w0.x & 0xFFFFu) | (w1.x << 16), (w0.x >> 16) | (w1.x & 0xFFFF0000u),
                                (w0.y & 0xFFFFu) | (w1.y << 16), (w0.y >> 16) | (w1.y & 0xFFFF0000u)};
#pragma unroll
        for (int e = 0; e < 4; ++e) *reinterpret_cast<unsigned*>(&sKh[(ch4 + e) * PK + 2 * rp]) = pr[e];
      } else {
        const float4 y0 = ws_unpack<EF>(kq[j][0]), y1 = ws_unpack<EF>(kq[j][1]);
        const float k0[4] = {y0.x, y0.y, y0.z, y0.w};
        const float k1[4] = {y1.x, y1.y, y1.z, y1.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          unsigned hh, ll;
          split2_bf16(k0[e], k1[e], hh, ll);     // rows 2 rp, 2 rp + 1 of channel ch4 + e
          *reinterpret_cast<unsigned*>(&sKh[(ch4 + e) * PK + 2 * rp]) = hh;
          *reinterpret_cast<unsigned*>(&sKl[(ch4 + e) * PK + 2 * rp]) = ll;
        }
      }
    }
    tU.template put<kPB>(sU);
    if (t < D) sGC[t] = pgc;
    if (n + 1 < a.NT) fetch(n + 1);
    __syncthreads();
    // v~ = U - W S (two accumulation chains over the D / 32 K blocks)
    if (vt_wave) {
      f4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < D / 32; ++kb) {
        const int ka = (16 * mt + r) * PW + 32 * kb + 8 * gq, kbb = (16 * ct + r) * PW + 32 * kb + 8 * gq;
        f4& acc = (kb & 1) ? acc1 : acc0;
        if constexpr (WS16) {
          acc = mma32(acc, *reinterpret_cast<const h8*>(&sWh[ka]), *reinterpret_cast<const h8*>(&sSh[kbb]));
        } else {
          const b8 ah = *reinterpret_cast<const b8*>(&sWh[ka]), al = *reinterpret_cast<const b8*>(&sWl[ka]);
          const b8 bh = *reinterpret_cast<const b8*>(&sSh[kbb]), bl = *reinterpret_cast<const b8*>(&sSl[kbb]);
          acc = mma3_bf16(acc, ah, al, bh, bl);
        }
      }
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = 16 * mt + 4 * gq + i, col = 16 * ct + r;
        v[i] = sU[row * kPB + col] - (acc0[i] + acc1[i]);
        a.VT[ch * kC * D + row * D + c0 + col] = v[i];
      }
      if constexpr (WS16) {
        *reinterpret_cast<uint2*>(&sVh[(16 * ct + r) * PK + 16 * mt + 4 * gq]) = pack_f16x4(f4{v[0], v[1], v[2], v[3]});
      } else {
        uint2 hh, ll;
        split2_bf16(v[0], v[1], hh.x, ll.x);
        split2_bf16(v[2], v[3], hh.y, ll.y);
        *reinterpret_cast<uint2*>(&sVh[(16 * ct + r) * PK + 16 * mt + 4 * gq]) = hh;
        *reinterpret_cast<uint2*>(&sVl[(16 * ct + r) * PK + 16 * mt + 4 * gq]) = ll;
      }
    }
    __syncthreads();
    // S <- gamma_C S + (lambda k)^T v~
#pragma unroll
    for (int q = 0; q < NST; ++q)
#pragma unroll
      for (int i = 0; i < 4; ++i) S[q][i] *= sGC[16 * rt[q] + 4 * gq + i];
#pragma unroll
    for (int kb = 0; kb < kC / 32; ++kb)
#pragma unroll
      for (int q = 0; q < NST; ++q) {
        const int ka = (16 * rt[q] + r) * PK + 32 * kb + 8 * gq, kbb = (16 * cs[q] + r) * PK + 32 * kb + 8 * gq;
        if constexpr (WS16)
          S[q] = mma32(S[q], *reinterpret_cast<const h8*>(&sKh[ka]), *reinterpret_cast<const h8*>(&sVh[kbb]));
        else
          S[q] = mma3_bf16(S[q], *reinterpret_cast<const b8*>(&sKh[ka]), *reinterpret_cast<const b8*>(&sKl[ka]),
                           *reinterpret_cast<const b8*>(&sVh[kbb]), *reinterpret_cast<const b8*>(&sVl[kbb]));
      }
    __syncthreads();
  }
}

// reverse scan of one (chain, 32-column slice): dS per chunk, dv~, dh0.
// The products run as bf16 hi/lo triples, as in the forward scan: lambda k
// and the state cotangent slice dS^T with the channel as the K index; Aqk^T,
// do^T, (gamma q)^T, W^T and (-dv~)^T with the chunk row as the K index
// (transposed stores of row pairs).  dS itself stays fp32 in the accumulators.
//
// A chunk step has three phases between workgroup barriers, and every
// operand has LDS of its own, so each is staged one phase or more before it
// is read, in the shadow of the products:
//   A  store dS, stage it as hi / lo planes; dS <- gamma_C dS + (gamma q)^T do
//      (everything it reads was staged during the previous chunk);
//   B  dv~ = (lambda k) dS + Aqk^T do on waves 0-7, then every wave stages
//      W^T of this chunk (read in C) and loads W of the next one;
//   C  dS <- dS - W^T dv~; every wave stages lambda k, Aqk^T, do^T,
//      (gamma q)^T and gamma_C of the next chunk (read in its A and B) and
//      loads the one after.
template <int D, int DO, bool WS16>
__global__ __launch_bounds__(ScanThreads<D>::value) void kda_bwd_rscan_kernel(BwdArgs a) {
  constexpr int EF = BwdWs<WS16>::F;    // lambda k, Aqk, gamma q, W in
  constexpr int NTH = ScanThreads<D>::value;
  constexpr int NS = D / 32;
  constexpr int NST = (D / 8) / (NTH / 64);
  static_assert(NST >= 1, "at least one state tile per wave");
  constexpr int PW = D + 8;     // bf16 pitch of rows whose K index is a channel
  constexpr int PK = kC + 8;    // bf16 pitch of rows whose K index is a chunk row
  __shared__ __attribute__((aligned(16))) __bf16 sLh[kC * PW], sLl[kC * PW];   // lambda k [64][D]
  __shared__ __attribute__((aligned(16))) __bf16 sAh[kC * PK], sAl[kC * PK];   // Aqk^T [64][64]
  __shared__ __attribute__((aligned(16))) __bf16 sQh[D * PK], sQl[D * PK];     // (gamma q)^T [D][64]
  __shared__ __attribute__((aligned(16))) __bf16 sWh[D * PK], sWl[D * PK];     // W^T [D][64]
  __shared__ __attribute__((aligned(16))) __bf16 sSh[32 * PW], sSl[32 * PW];   // dS^T [32][D]
  __shared__ __attribute__((aligned(16))) __bf16 sOh[32 * PK], sOl[32 * PK];   // do^T [32][64]
  __shared__ __attribute__((aligned(16))) __bf16 sVh[32 * PK], sVl[32 * PK];   // (-dv~)^T [32][64]
  __shared__ float sGC[D];
  const int t = threadIdx.x, wv = t >> 6, l = t & 63, r = l & 15, gq = l >> 4;
  const int H = a.H;
  int chain, split;
  if (!scan_slot<NS>(a.B * H, chain, split)) return;   // uniform per workgroup
  const int b = chain / H, h = chain - b * H;
  const int c0 = 32 * split;
  const int mt = wv >> 1, ct = wv & 1;                  // this wave's dv~ tile (waves 0-7: 8 tiles)
  const bool vt_wave = wv < 8;
  const int mts = __builtin_amdgcn_readfirstlane(mt);
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
  // Operands in registers between their loads and their staging, one set
  // each: a set is reloaded right after it is staged, so every load has a
  // whole chunk step to arrive.  The do slice is held as loaded (raw words),
  // so that no wait falls at its load.
  Tile<kC, D, NTH, EF> tL;
  TTile<kC, kScanThreads, EF> tA;   // threads t < kScanThreads
  TTile<D, NTH, EF> tQ, tW;
  const bool a_thread = t < kScanThreads;
  float pgc;   // gamma_C of the chunk (every thread; t < D stages it)
  // do^T of the slice, spread over every thread: thread t holds rows 2 rp,
  // 2 rp + 1 of the DCPT columns c0 + DCPT cg .. (consecutive threads at
  // consecutive columns; rows past the chunk's end are loaded from row 0 and
  // zeroed where staged), as raw words
  constexpr int DCPT = (kC * 32) / 2 / NTH;   // columns per thread
  constexpr int DCG = 32 / DCPT;              // column groups
  static_assert(DCPT >= 1 && DCPT <= 2 && DCG * DCPT == 32 && 2 * DCG * 32 == 2 * NTH, "do slice mapping");
  uint32_t pdo[2][DCPT];
  const int dcg = t % DCG, drp = t / DCG;
  auto do_val = [&](uint32_t w) -> float {
    if constexpr (DO == 0) return __uint_as_float(w);
    else if constexpr (DO == 1) return __uint_as_float(w << 16);
    else return f16bits_to_f32(static_cast<u16>(w));
  };
  auto chead = [&](int n) { return (static_cast<int64_t>(b) * a.NT + n) * H + h; };
  auto fetch_a = [&](int n) {   // lambda k, Aqk, gamma q, gamma_C and do of chunk n
    const int u = b * a.NT + n;
    const int64_t ch = chead(n);
    tL.fetch(ws_at<EF>(a.KL, ch * kC * D), D, 0);
    if (a_thread) tA.fetch(ws_at<EF>(a.AQ, ch * kC * kC), kC, 0);
    tQ.fetch(ws_at<EF>(a.QG, ch * kC * D), D, 0);
    pgc = a.GCV[ch * D + (t & (D - 1))];
    const ChunkRows crn = chunk_rows(a, u);
#pragma unroll
    for (int y = 0; y < 2; ++y) {
      const int row = 2 * drp + y;
      const int64_t i = ((crn.row0 + (row < crn.len ? row : 0)) * H + h) * D + c0 + DCPT * dcg;
#pragma unroll
      for (int e = 0; e < DCPT; ++e) {
        if constexpr (DO == 0) pdo[y][e] = static_cast<const uint32_t*>(a.dout)[i + e];
        else pdo[y][e] = static_cast<const u16*>(a.dout)[i + e];
      }
    }
  };
  auto put_a = [&](int n) {     // ... staged for chunk n
    const ChunkRows crn = chunk_rows(a, b * a.NT + n);
    put_hl<PW>(tL, sLh, sLl);
    if (a_thread) tA.template put_hl<PK>(sAh, sAl);
    tQ.template put_hl<PK>(sQh, sQl);
    const bool ok0 = 2 * drp < crn.len, ok1 = 2 * drp + 1 < crn.len;
#pragma unroll
    for (int e = 0; e < DCPT; ++e) {
      unsigned hh, ll;
      split2_bf16(ok0 ? do_val(pdo[0][e]) : 0.f, ok1 ? do_val(pdo[1][e]) : 0.f, hh, ll);
      *reinterpret_cast<unsigned*>(&sOh[(DCPT * dcg + e) * PK + 2 * drp]) = hh;
      *reinterpret_cast<unsigned*>(&sOl[(DCPT * dcg + e) * PK + 2 * drp]) = ll;
    }
    if (t < D) sGC[t] = pgc;
  };
  if (a.NT > 0) {
    fetch_a(a.NT - 1);
    tW.fetch(ws_at<EF>(a.WM, chead(a.NT - 1) * kC * D), D, 0);
    put_a(a.NT - 1);
    if (a.NT > 1) fetch_a(a.NT - 2);
    __syncthreads();
  }
  for (int n = a.NT - 1; n >= 0; --n) {
    const int64_t ch = chead(n);
    // ---- A: store and stage dS; dS <- gamma_C dS + (gamma q)^T do
#pragma unroll
    for (int q = 0; q < NST; ++q) {
      const int m0 = 16 * rt[q] + 4 * gq, col = 16 * cs[q] + r;
#pragma unroll
      for (int i = 0; i < 4; ++i) a.DS[ch * D * D + (m0 + i) * D + c0 + col] = dS[q][i];
      uint2 hh, ll;
      split2_bf16(dS[q][0], dS[q][1], hh.x, ll.x);
      split2_bf16(dS[q][2], dS[q][3], hh.y, ll.y);
      *reinterpret_cast<uint2*>(&sSh[col * PW + m0]) = hh;
      *reinterpret_cast<uint2*>(&sSl[col * PW + m0]) = ll;
    }
#pragma unroll
    for (int q = 0; q < NST; ++q)
#pragma unroll
      for (int i = 0; i < 4; ++i) dS[q][i] *= sGC[16 * rt[q] + 4 * gq + i];
#pragma unroll
    for (int kb = 0; kb < kC / 32; ++kb)
#pragma unroll
      for (int q = 0; q < NST; ++q) {
        const int ka = (16 * rt[q] + r) * PK + 32 * kb + 8 * gq, kbb = (16 * cs[q] + r) * PK + 32 * kb + 8 * gq;
        dS[q] = mma3_bf16(dS[q], *reinterpret_cast<const b8*>(&sQh[ka]), *reinterpret_cast<const b8*>(&sQl[ka]),
                          *reinterpret_cast<const b8*>(&sOh[kbb]), *reinterpret_cast<const b8*>(&sOl[kbb]));
      }
    __syncthreads();
    // ---- B: dv~ = (lambda k) dS + Aqk^T do; Aqk[j][m] is zero for j < m,
    // so row tile mt starts at the K block holding row 16 mt
    if (vt_wave) {
      f4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < D / 32; ++kb) {
        const int ka = (16 * mt + r) * PW + 32 * kb + 8 * gq, kbb = (16 * ct + r) * PW + 32 * kb + 8 * gq;
        acc0 = mma3_bf16(acc0, *reinterpret_cast<const b8*>(&sLh[ka]), *reinterpret_cast<const b8*>(&sLl[ka]),
                         *reinterpret_cast<const b8*>(&sSh[kbb]), *reinterpret_cast<const b8*>(&sSl[kbb]));
      }
      for (int kb = mts >> 1; kb < kC / 32; ++kb) {
        const int ka = (16 * mt + r) * PK + 32 * kb + 8 * gq, kbb = (16 * ct + r) * PK + 32 * kb + 8 * gq;
        acc1 = mma3_bf16(acc1, *reinterpret_cast<const b8*>(&sAh[ka]), *reinterpret_cast<const b8*>(&sAl[ka]),
                         *reinterpret_cast<const b8*>(&sOh[kbb]), *reinterpret_cast<const b8*>(&sOl[kbb]));
      }
      float* DVT = a.DVT + ch * kC * D;
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[i] = acc0[i] + acc1[i];
        DVT[(16 * mt + 4 * gq + i) * D + c0 + 16 * ct + r] = v[i];
      }
      uint2 hh, ll;
      split2_bf16(-v[0], -v[1], hh.x, ll.x);
      split2_bf16(-v[2], -v[3], hh.y, ll.y);
      *reinterpret_cast<uint2*>(&sVh[(16 * ct + r) * PK + 16 * mt + 4 * gq]) = hh;
      *reinterpret_cast<uint2*>(&sVl[(16 * ct + r) * PK + 16 * mt + 4 * gq]) = ll;
    }
    tW.template put_hl<PK>(sWh, sWl);
    if (n > 0) tW.fetch(ws_at<EF>(a.WM, chead(n - 1) * kC * D), D, 0);
    __syncthreads();
    // ---- C: dS <- dS - W^T dv~; the next chunk's lambda k, Aqk^T, do^T,
    // (gamma q)^T and gamma_C staged while the products run
#pragma unroll
    for (int kb = 0; kb < kC / 32; ++kb)
#pragma unroll
      for (int q = 0; q < NST; ++q) {
        const int ka = (16 * rt[q] + r) * PK + 32 * kb + 8 * gq, kbb = (16 * cs[q] + r) * PK + 32 * kb + 8 * gq;
        dS[q] = mma3_bf16(dS[q], *reinterpret_cast<const b8*>(&sWh[ka]), *reinterpret_cast<const b8*>(&sWl[ka]),
                          *reinterpret_cast<const b8*>(&sVh[kbb]), *reinterpret_cast<const b8*>(&sVl[kbb]));
      }
    if (n > 0) {
      put_a(n - 1);
      if (n > 1) fetch_a(n - 2);
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
// Reverse scan for 16-bit inputs: one workgroup per (chain, 32-column slice),
// two compute waves (one 16-column value tile each) and four producer waves,
// as the forward's state kernel.  Each compute wave owns its tile's columns of
// dS for every channel, so a chunk step needs no exchange between waves:
//   dv~ = (lambda k) dS' + Aqk^T do,  dS <- gamma_C dS + (gamma q)^T do - W^T dv~
// with the forward-side operands (lambda k, Aqk^T, (gamma q)^T, W^T) as the
// prep kernel's fp16 A fragments, staged by the producers into one of two LDS
// buffers two chunks ahead, and the cotangent operands (dS', do, dv~) as B
// fragments formed in registers.  A cotangent's scale is the caller's, so
// each B column is scaled by a power of two that brings its largest element
// to [2^14, 2^15) and split into fp16 hi + lo (about 22 significant bits,
// fp16's range no limit); each product is two fp16 MFMAs per K step, and the
// column's scale is taken off the accumulator (every lane's D column is its
// own B column).  One barrier per chunk step.
// ---------------------------------------------------------------------------
constexpr int kRsProducers = 4;

template <int D>
struct RsLayout {
  static constexpr int NFL = 4 * (D / 32);         // lambda k fragments (row tile, K step over channels)
  static constexpr int NFA = 6;                    // Aqk^T fragments
  static constexpr int NFQ = 2 * (D / 16);         // (gamma q)^T fragments (channel tile, K step over rows)
  static constexpr int OFF_A = NFL;                // in 1 KiB fragments
  static constexpr int OFF_Q = OFF_A + NFA;
  static constexpr int OFF_W = OFF_Q + NFQ;
  static constexpr int NF = OFF_W + NFQ;           // fragments per chunk
  static constexpr int OFF_GC = NF * 1024;         // gamma_C, D floats
  static constexpr int OFF_DO = OFF_GC + 4 * D;    // do B fragments [K step][value tile][64][8] fp32
  static constexpr int BYTES = OFF_DO + 2 * 2 * 64 * 8 * 4;
  static constexpr int SROW = 36;                  // staging row stride in floats (rows 4 apart land 16 banks apart)
  static constexpr int STG = kC * SROW * 4;        // dv~ of the slice, fp32 [64][32], stored a step later
};

// One chunk's share of producer P: every kRsProducers-th fragment, two
// 16-byte pieces of the do rows, and (last producer) gamma_C.
template <int D, int P>
struct RsRegs {
  static constexpr int NFP = (RsLayout<D>::NF - P + kRsProducers - 1) / kRsProducers;
  u32x4 f[NFP];
  uint4 d[2];
  u32x4 g;
};

template <int D, int DO, int P>
__device__ __forceinline__ void rs_load(const BwdArgs& a, int b, int n, int h, int c0, int l, RsRegs<D, P>& R) {
  typedef RsLayout<D> LY;
  const int H = a.H;
  const int64_t ch = (static_cast<int64_t>(b) * a.NT + n) * H + h;
#pragma unroll
  for (int k = 0; k < RsRegs<D, P>::NFP; ++k) {
    const int f = P + kRsProducers * k;
    const _Float16* src;
    if (f < LY::OFF_A) src = static_cast<const _Float16*>(a.FL) + (ch * LY::NFL + f) * 512;
    else if (f < LY::OFF_Q) src = static_cast<const _Float16*>(a.FA) + (ch * LY::NFA + (f - LY::OFF_A)) * 512;
    else if (f < LY::OFF_W) src = static_cast<const _Float16*>(a.FQ) + (ch * LY::NFQ + (f - LY::OFF_Q)) * 512;
    else src = static_cast<const _Float16*>(a.FW) + (ch * LY::NFQ + (f - LY::OFF_W)) * 512;
    R.f[k] = *reinterpret_cast<const u32x4*>(src + l * 8);
  }
  // do rows of the slice: 64 rows x 32 columns = 512 pieces of four columns,
  // 128 per producer; rows past the chunk's end load row 0 (zeroed when written)
  const ChunkRows cr = chunk_rows(a, b * a.NT + n);
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int pc = 128 * P + 64 * k + l, row = pc >> 3, c4 = pc & 7;
    const int64_t i = ((cr.row0 + (row < cr.len ? row : 0)) * H + h) * D + c0 + 4 * c4;
    if constexpr (DO == 0) R.d[k] = *reinterpret_cast<const uint4*>(static_cast<const float*>(a.dout) + i);
    else {
      const uint2 w = *reinterpret_cast<const uint2*>(static_cast<const u16*>(a.dout) + i);
      R.d[k] = uint4{w.x, w.y, 0u, 0u};
    }
  }
  if constexpr (P == kRsProducers - 1) {
    R.g = u32x4{0, 0, 0, 0};
    if (l < D / 4) R.g = *reinterpret_cast<const u32x4*>(a.GCV + ch * D + 4 * l);
  }
}

template <int D, int DO, int P>
__device__ __forceinline__ void rs_write(unsigned char* dst, const BwdArgs& a, int b, int n, int l,
                                         const RsRegs<D, P>& R) {
  typedef RsLayout<D> LY;
#pragma unroll
  for (int k = 0; k < RsRegs<D, P>::NFP; ++k)
    *reinterpret_cast<u32x4*>(dst + (P + kRsProducers * k) * 1024 + l * 16) = R.f[k];
  const int len = chunk_rows(a, b * a.NT + n).len;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int pc = 128 * P + 64 * k + l, row = pc >> 3, c4 = pc & 7;
    float x[4];
    if constexpr (DO == 0) {
      x[0] = __uint_as_float(R.d[k].x); x[1] = __uint_as_float(R.d[k].y);
      x[2] = __uint_as_float(R.d[k].z); x[3] = __uint_as_float(R.d[k].w);
    } else {
      const f4 v = unpack4<1>(uint2{R.d[k].x, R.d[k].y});
      x[0] = v[0]; x[1] = v[1]; x[2] = v[2]; x[3] = v[3];
    }
    // B fragment (K step row / 32, value tile col / 16), lane (col % 16) +
    // 16 ((row % 16) / 4), element (row % 4) + 4 ((row % 32) / 16)
    const int kb = row >> 5, rr = row & 31;
    const int lane_hi = 16 * ((rr & 15) >> 2), e = (rr & 3) + 4 * (rr >> 4);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int col = 4 * c4 + i;
      float* p = reinterpret_cast<float*>(dst + LY::OFF_DO) +
                 ((kb * 2 + (col >> 4)) * 64 + (col & 15) + lane_hi) * 8 + e;
      *p = (row < len) ? x[i] : 0.f;
    }
  }
  if constexpr (P == kRsProducers - 1)
    if (l < D / 4) *reinterpret_cast<u32x4*>(dst + LY::OFF_GC + l * 16) = R.g;
}

// Producer P's share of chunk n's dv~ rows from the staging area (64 rows x
// 8 pieces of four columns, 16-byte stores).
template <int D, int P>
__device__ __forceinline__ void rs_store(const BwdArgs& a, const unsigned char* stg, int b, int n, int h, int c0,
                                         int l) {
  const int64_t ch = (static_cast<int64_t>(b) * a.NT + n) * a.H + h;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int pc = 128 * P + 64 * k + l, row = pc >> 3, c4 = pc & 7;
    const f4 v = *reinterpret_cast<const f4*>(stg + (row * RsLayout<D>::SROW + 4 * c4) * 4);
    *reinterpret_cast<f4*>(a.DVT + ch * kC * D + row * D + c0 + 4 * c4) = v;
  }
}

template <int D, int DO, int P>
__device__ __forceinline__ void rs_producer(const BwdArgs& a, unsigned char (*buf)[RsLayout<D>::BYTES],
                                            unsigned char (*stg)[RsLayout<D>::STG], int b, int h, int c0) {
  const int l = threadIdx.x & 63;
  const int NT = a.NT;
  RsRegs<D, P> R0, R1;
  // step s works on chunk NT - 1 - s
  rs_load<D, DO, P>(a, b, NT - 1, h, c0, l, R0);
  rs_load<D, DO, P>(a, b, max(NT - 2, 0), h, c0, l, R1);
  rs_write<D, DO, P>(buf[0], a, b, NT - 1, l, R0);
  lds_barrier();   // chunk of step 0 staged
  auto step = [&](int s, RsRegs<D, P>& Rn, RsRegs<D, P>& Rn1) {
    // store step s-1's dv~; Rn held step s's chunk (in LDS since the last
    // barrier): load step s+2's; write step s+1's from Rn1 (loaded a step
    // earlier) into the free buffer
    if (s > 0) rs_store<D, P>(a, stg[(s - 1) & 1], b, NT - s, h, c0, l);
    rs_load<D, DO, P>(a, b, max(NT - 3 - s, 0), h, c0, l, Rn);
    if (s + 1 < NT) rs_write<D, DO, P>(buf[(s + 1) & 1], a, b, NT - 2 - s, l, Rn1);
    lds_barrier();
  };
  int s = 0;
  for (; s + 1 < NT; s += 2) {
    step(s, R0, R1);
    step(s + 1, R1, R0);
  }
  if (s < NT) step(s, R0, R1);
  rs_store<D, P>(a, stg[(NT - 1) & 1], b, 0, h, c0, l);
  wait_vmem_all();
}

// A column's scale 2^e, e = 15 - exponent(largest |x|), so the largest
// scaled element lies in [2^14, 2^15); e is at most 126 (a column below
// 2^-111 is scaled less than that, which only costs it relative precision it
// cannot use), and at least 15 - 128 for finite x, so 2^e and 2^-e are normal
// floats: the scale and its inverse are exact multipliers.
struct RsScale {
  float up, down;
};
__device__ __forceinline__ RsScale rs_col_scale(float m) {
  const int e = min(15 - __builtin_amdgcn_frexp_expf(m), 126);
  return RsScale{__builtin_amdgcn_ldexpf(1.f, e), __builtin_amdgcn_ldexpf(1.f, -e)};
}
// eight B values, scaled, as fp16 hi + lo
__device__ __forceinline__ void rs_split(const float (&x)[8], float up, h8& hi, h8& lo) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float y = x[i] * up;
    hi[i] = static_cast<_Float16>(y);
    lo[i] = static_cast<_Float16>(y - static_cast<float>(hi[i]));
  }
}
// largest |x| of a column over the four lanes (gq) that hold it
__device__ __forceinline__ float rs_col_max(float m) {
  m = fmaxf(m, __shfl_xor(m, 16, 64));
  return fmaxf(m, __shfl_xor(m, 32, 64));
}

template <int D, int W>
__device__ __forceinline__ void rs_chain(const BwdArgs& a, unsigned char (*buf)[RsLayout<D>::BYTES],
                                         unsigned char (*stg)[RsLayout<D>::STG], int b, int h, int chain, int c0) {
  typedef RsLayout<D> LY;
  constexpr int NT_ = D / 16;   // channel tiles
  constexpr int NJ = D / 32;    // K steps over the channels
  const int l = threadIdx.x & 63, r = l & 15, gq = l >> 4;
  const int col = c0 + 16 * W + r;   // this lane's value column
  const int NT = a.NT;
  f4 dS[NT_];
  const int64_t sbase = static_cast<int64_t>(chain) * D * D + (4 * gq) * D + col;   // + (16 dt + i) D
#pragma unroll
  for (int dt = 0; dt < NT_; ++dt)
#pragma unroll
    for (int i = 0; i < 4; ++i) dS[dt][i] = (a.dht != nullptr) ? a.dht[sbase + (16 * dt + i) * D] : 0.f;
  lds_barrier();   // chunk of step 0 staged by the producers
  for (int s = 0; s < NT; ++s) {
    const int n = NT - 1 - s;
    const int64_t ch = (static_cast<int64_t>(b) * NT + n) * a.H + h;
    const unsigned char* cur = buf[s & 1];
    auto frag = [&](int f) { return *reinterpret_cast<const h8*>(cur + f * 1024 + l * 16); };
    // the dv~ products' A fragments and the do B values, read ahead of the
    // arithmetic that forms dS' and do's B fragments
    h8 AL[4][NJ], AA[6];
#pragma unroll
    for (int ct = 0; ct < 4; ++ct)
#pragma unroll
      for (int j = 0; j < NJ; ++j) AL[ct][j] = frag(ct * NJ + j);
#pragma unroll
    for (int f = 0; f < 6; ++f) AA[f] = frag(LY::OFF_A + f);
    float dov[2][8];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const float* p = reinterpret_cast<const float*>(cur + LY::OFF_DO) + ((kb * 2 + W) * 64 + l) * 8;
      const f4 lo = *reinterpret_cast<const f4*>(p), hi4 = *reinterpret_cast<const f4*>(p + 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) { dov[kb][i] = lo[i]; dov[kb][4 + i] = hi4[i]; }
    }
    // (the reads stay here, ahead of the arithmetic below)
    __builtin_amdgcn_sched_barrier(0);
    // dS' (the cotangent of the state this chunk leaves) to the workspace
    float* const dsp = a.DS + ch * D * D + (4 * gq) * D + col;
#pragma unroll
    for (int dt = 0; dt < NT_; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) dsp[(16 * dt + i) * D] = dS[dt][i];
    // B fragments: dS' over the channels, do over the rows
    float m1 = 0.f;
#pragma unroll
    for (int dt = 0; dt < NT_; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) m1 = fmaxf(m1, fabsf(dS[dt][i]));
    const RsScale e1 = rs_col_scale(rs_col_max(m1));
    h8 Sh[NJ], Sl[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const float x[8] = {dS[2 * j][0], dS[2 * j][1], dS[2 * j][2], dS[2 * j][3],
                          dS[2 * j + 1][0], dS[2 * j + 1][1], dS[2 * j + 1][2], dS[2 * j + 1][3]};
      rs_split(x, e1.up, Sh[j], Sl[j]);
    }
    float m2 = 0.f;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < 8; ++i) m2 = fmaxf(m2, fabsf(dov[kb][i]));
    const RsScale e2 = rs_col_scale(rs_col_max(m2));
    h8 Dh[2], Dl[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) rs_split(dov[kb], e2.up, Dh[kb], Dl[kb]);
    // dv~ = (lambda k) dS' + Aqk^T do, row tile ct
    f4 p1[4], p2[4];
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      p1[ct] = f4{0.f, 0.f, 0.f, 0.f};
      p2[ct] = f4{0.f, 0.f, 0.f, 0.f};
    }
    // (consecutive MFMAs feed different accumulators)
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) p1[ct] = mma32(p1[ct], AL[ct][j], Sh[j]);
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) p1[ct] = mma32(p1[ct], AL[ct][j], Sl[j]);
    }
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int hl = 0; hl < 2; ++hl)
#pragma unroll
        for (int ct = 0; ct < 4; ++ct) {
          if (ct >= 2 && kb == 0) continue;   // query rows 0..31 hold no pair with keys 32..63
          p2[ct] = mma32(p2[ct], AA[fa_frag(ct, kb)], hl ? Dl[kb] : Dh[kb]);
        }
    // the dS update's (gamma q)^T fragments; (gamma q)^T do does not wait for dv~
    h8 AQ[NT_][2];
#pragma unroll
    for (int dt = 0; dt < NT_; ++dt)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) AQ[dt][kb] = frag(LY::OFF_Q + 2 * dt + kb);
    f4 pq[NT_];
#pragma unroll
    for (int dt = 0; dt < NT_; ++dt) pq[dt] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int hl = 0; hl < 2; ++hl)
#pragma unroll
        for (int dt = 0; dt < NT_; ++dt) pq[dt] = mma32(pq[dt], AQ[dt][kb], hl ? Dl[kb] : Dh[kb]);
    h8 AW[NT_][2];
#pragma unroll
    for (int dt = 0; dt < NT_; ++dt)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) AW[dt][kb] = frag(LY::OFF_W + 2 * dt + kb);
    f4 dvt[4];
#pragma unroll
    for (int ct = 0; ct < 4; ++ct)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        dvt[ct][i] = fmaf(p1[ct][i], e1.down, p2[ct][i] * e2.down);
    float* const dvo = reinterpret_cast<float*>(stg[s & 1]);   // stored by the producers a step later
#pragma unroll
    for (int ct = 0; ct < 4; ++ct)
#pragma unroll
      for (int i = 0; i < 4; ++i) dvo[(16 * ct + 4 * gq + i) * LY::SROW + 16 * W + r] = dvt[ct][i];
    // dv~ as B fragments over the rows
    float m3 = 0.f;
#pragma unroll
    for (int ct = 0; ct < 4; ++ct)
#pragma unroll
      for (int i = 0; i < 4; ++i) m3 = fmaxf(m3, fabsf(dvt[ct][i]));
    const RsScale e3 = rs_col_scale(rs_col_max(m3));
    h8 Vh[2], Vl[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const float x[8] = {dvt[2 * kb][0], dvt[2 * kb][1], dvt[2 * kb][2], dvt[2 * kb][3],
                          dvt[2 * kb + 1][0], dvt[2 * kb + 1][1], dvt[2 * kb + 1][2], dvt[2 * kb + 1][3]};
      rs_split(x, e3.up, Vh[kb], Vl[kb]);
    }
    // dS <- gamma_C dS + (gamma q)^T do - W^T dv~, channel tile dt
    f4 pw[NT_];
#pragma unroll
    for (int dt = 0; dt < NT_; ++dt) pw[dt] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int hl = 0; hl < 2; ++hl)
#pragma unroll
        for (int dt = 0; dt < NT_; ++dt) pw[dt] = mma32(pw[dt], AW[dt][kb], hl ? Vl[kb] : Vh[kb]);
#pragma unroll
    for (int dt = 0; dt < NT_; ++dt) {
      const f4 gc = *reinterpret_cast<const f4*>(cur + LY::OFF_GC + (16 * dt + 4 * gq) * 4);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        dS[dt][i] = fmaf(-pw[dt][i], e3.down, fmaf(pq[dt][i], e2.down, dS[dt][i] * gc[i]));
    }
    lds_barrier();   // this buffer is free, the next one staged
  }
  if (a.dh0 != nullptr) {
#pragma unroll
    for (int dt = 0; dt < NT_; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) a.dh0[sbase + (16 * dt + i) * D] = dS[dt][i];
  }
}

template <int D, int DO>
__global__ __launch_bounds__(64 * (2 + kRsProducers), 1) void kda_bwd_rscan16_kernel(BwdArgs a) {
  constexpr int NS = D / 32;
  __shared__ __attribute__((aligned(16))) unsigned char buf[2][RsLayout<D>::BYTES];
  __shared__ __attribute__((aligned(16))) unsigned char stg[2][RsLayout<D>::STG];
  int chain, split;
  if (!scan_slot<NS>(a.B * a.H, chain, split)) return;   // uniform per workgroup
  const int b = chain / a.H, h = chain - b * a.H;
  const int c0 = 32 * split;
  const int wave = threadIdx.x >> 6;
  switch (wave) {
    case 0: rs_chain<D, 0>(a, buf, stg, b, h, chain, c0); break;
    case 1: rs_chain<D, 1>(a, buf, stg, b, h, chain, c0); break;
    case 2: rs_producer<D, DO, 0>(a, buf, stg, b, h, c0); break;
    case 3: rs_producer<D, DO, 1>(a, buf, stg, b, h, c0); break;
    case 4: rs_producer<D, DO, 2>(a, buf, stg, b, h, c0); break;
    default: rs_producer<D, DO, 3>(a, buf, stg, b, h, c0); break;
  }
}

// ---------------------------------------------------------------------------
// Forward state scan for 16-bit inputs, in the form of the reverse scan above
// (and of the forward's state kernel): per (chain, 32-column slice) two
// compute waves own a 16-column tile of S each,
//   v~ = U - W S,  S <- gamma_C S + (lambda k)^T v~,
// with W and (lambda k)^T as the prep kernel's fp16 A fragments and S, v~
// handed to the matrix cores as fp16 (the forward kernels' operands); four
// producer waves stage W, (lambda k)^T, the slice's U tiles (fp32) and gamma_C
// two chunks ahead.  Each chunk's incoming S is stored fp16 row-major: the
// D-layout tile read as an A fragment is S^T, and its product with the
// identity puts four consecutive columns of one row of S in each lane.  The
// compute waves write S and v~ into a staging area and the producers store
// them with 16-byte stores a step later, so the compute waves issue no global
// memory operation inside the chunk loop.
// ---------------------------------------------------------------------------
constexpr int kFsProducers = 4;

template <int D>
struct FsLayout {
  static constexpr int NFW = 4 * (D / 32);         // W fragments (row tile, K step over channels)
  static constexpr int NFL = 2 * (D / 16);         // (lambda k)^T fragments (channel tile, K step over rows)
  static constexpr int NF = NFW + NFL;             // 1 KiB fragments
  static constexpr int OFF_U = NF * 1024;          // U tiles [row tile][value tile of the slice][64][4] fp32
  static constexpr int NU = 4 * 2;
  static constexpr int OFF_GC = OFF_U + NU * 1024; // gamma_C, D floats
  static constexpr int BYTES = OFF_GC + 4 * D;
  // the compute waves' outputs of a chunk, stored by the producers a step
  // later: S fp16 [D][32], v~ fp32 [64][32] of the slice
  static constexpr int STG_VT = D * 32 * 2;
  static constexpr int STG = STG_VT + kC * 32 * 4;
};

// Producer P's share of a chunk: every kFsProducers-th fragment, two four-
// column pieces of the slice's U rows (64 rows x 8 pieces, 128 per producer)
// and (last producer) gamma_C.
template <int D, int P>
struct FsRegs {
  static constexpr int NFP = (FsLayout<D>::NF - P + kFsProducers - 1) / kFsProducers;
  u32x4 f[NFP];
  f4 u[2];
  u32x4 g;
};

template <int D, int P>
__device__ __forceinline__ void fs_load(const BwdArgs& a, int b, int n, int h, int split, int l, FsRegs<D, P>& R) {
  typedef FsLayout<D> LY;
  const int64_t ch = (static_cast<int64_t>(b) * a.NT + n) * a.H + h;
#pragma unroll
  for (int k = 0; k < FsRegs<D, P>::NFP; ++k) {
    const int f = P + kFsProducers * k;
    const _Float16* src = (f < LY::NFW) ? static_cast<const _Float16*>(a.FWN) + (ch * LY::NFW + f) * 512
                                        : static_cast<const _Float16*>(a.FLT) + (ch * LY::NFL + (f - LY::NFW)) * 512;
    R.f[k] = *reinterpret_cast<const u32x4*>(src + l * 8);
  }
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int pc = 128 * P + 64 * k + l, row = pc >> 3, c4 = pc & 7;
    R.u[k] = *reinterpret_cast<const f4*>(a.UM + ch * kC * D + row * D + 32 * split + 4 * c4);
  }
  if constexpr (P == kFsProducers - 1) {
    R.g = u32x4{0, 0, 0, 0};
    if (l < D / 4) R.g = *reinterpret_cast<const u32x4*>(a.GCV + ch * D + 4 * l);
  }
}

template <int D, int P>
__device__ __forceinline__ void fs_write(unsigned char* dst, int l, const FsRegs<D, P>& R) {
  typedef FsLayout<D> LY;
#pragma unroll
  for (int k = 0; k < FsRegs<D, P>::NFP; ++k)
    *reinterpret_cast<u32x4*>(dst + (P + kFsProducers * k) * 1024 + l * 16) = R.f[k];
  // U piece (row, four columns) into the D-layout tiles [row tile][value
  // tile]: lane (col % 16) + 16 ((row % 16) / 4), element row % 4
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int pc = 128 * P + 64 * k + l, row = pc >> 3, c4 = pc & 7;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int col = 4 * c4 + i;
      reinterpret_cast<float*>(dst + LY::OFF_U)[(((row >> 4) * 2 + (col >> 4)) * 64 + (col & 15) +
                                                 16 * ((row & 15) >> 2)) * 4 + (row & 3)] = R.u[k][i];
    }
  }
  if constexpr (P == kFsProducers - 1)
    if (l < D / 4) *reinterpret_cast<u32x4*>(dst + LY::OFF_GC + l * 16) = R.g;
}

// Producer P's share of chunk n's outputs from the staging area: 16-byte
// pieces of the S rows (D rows x 4) and of the v~ rows (64 rows x 8).
template <int D, int P>
__device__ __forceinline__ void fs_store(const BwdArgs& a, const unsigned char* stg, int b, int n, int h, int split,
                                         int l) {
  typedef FsLayout<D> LY;
  const int64_t ch = (static_cast<int64_t>(b) * a.NT + n) * a.H + h;
  constexpr int NSP = D * 4 / (64 * kFsProducers);   // S pieces per lane
#pragma unroll
  for (int k = 0; k < NSP; ++k) {
    const int pc = 64 * (NSP * P + k) + l, row = pc >> 2, c8 = pc & 3;
    const uint4 v = *reinterpret_cast<const uint4*>(stg + (row * 32 + 8 * c8) * 2);
    *reinterpret_cast<uint4*>(reinterpret_cast<u16*>(a.SI) + ch * D * D + row * D + 32 * split + 8 * c8) = v;
  }
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int pc = 128 * P + 64 * k + l, row = pc >> 3, c4 = pc & 7;
    const f4 v = *reinterpret_cast<const f4*>(stg + LY::STG_VT + (row * 32 + 4 * c4) * 4);
    *reinterpret_cast<f4*>(a.VT + ch * kC * D + row * D + 32 * split + 4 * c4) = v;
  }
}

template <int D, int P>
__device__ __forceinline__ void fs_producer(const BwdArgs& a, unsigned char (*buf)[FsLayout<D>::BYTES],
                                            unsigned char (*stg)[FsLayout<D>::STG], int b, int h, int split) {
  const int l = threadIdx.x & 63;
  const int NT = a.NT;
  FsRegs<D, P> R0, R1;
  fs_load<D, P>(a, b, 0, h, split, l, R0);
  fs_load<D, P>(a, b, min(1, NT - 1), h, split, l, R1);
  fs_write<D, P>(buf[0], l, R0);
  lds_barrier();   // chunk 0 staged
  auto step = [&](int n, FsRegs<D, P>& Rn, FsRegs<D, P>& Rn1) {
    if (n > 0) fs_store<D, P>(a, stg[(n - 1) & 1], b, n - 1, h, split, l);
    fs_load<D, P>(a, b, min(n + 2, NT - 1), h, split, l, Rn);
    if (n + 1 < NT) fs_write<D, P>(buf[(n + 1) & 1], l, Rn1);
    lds_barrier();
  };
  int n = 0;
  for (; n + 1 < NT; n += 2) {
    step(n, R0, R1);
    step(n + 1, R1, R0);
  }
  if (n < NT) step(n, R0, R1);
  fs_store<D, P>(a, stg[(NT - 1) & 1], b, NT - 1, h, split, l);
  wait_vmem_all();
}

template <int D, int W>
__device__ __forceinline__ void fs_chain(const BwdArgs& a, unsigned char (*buf)[FsLayout<D>::BYTES],
                                         unsigned char (*stg)[FsLayout<D>::STG], int b, int h, int chain, int c0) {
  typedef FsLayout<D> LY;
  constexpr int NT_ = D / 16;
  constexpr int NJ = D / 32;
  const int l = threadIdx.x & 63, r = l & 15, gq = l >> 4;
  const int col = c0 + 16 * W + r;
  const int NT = a.NT;
  f4 S[NT_];
#pragma unroll
  for (int dt = 0; dt < NT_; ++dt)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      S[dt][i] = (a.h0 != nullptr) ? a.h0[(static_cast<int64_t>(chain) * D + 16 * dt + 4 * gq + i) * D + col] : 0.f;
  h4 ident;
#pragma unroll
  for (int i = 0; i < 4; ++i) ident[i] = static_cast<_Float16>((4 * gq + i == r) ? 1.f : 0.f);
  lds_barrier();   // chunk 0 staged by the producers
  for (int n = 0; n < NT; ++n) {
    const int64_t ch = (static_cast<int64_t>(b) * NT + n) * a.H + h;
    const unsigned char* cur = buf[n & 1];
    auto frag = [&](int f) { return *reinterpret_cast<const h8*>(cur + f * 1024 + l * 16); };
    h8 AW[4][NJ];
#pragma unroll
    for (int ct = 0; ct < 4; ++ct)
#pragma unroll
      for (int j = 0; j < NJ; ++j) AW[ct][j] = frag(ct * NJ + j);
    f4 Ut[4];
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) Ut[ct] = *reinterpret_cast<const f4*>(cur + LY::OFF_U + (2 * ct + W) * 1024 + l * 16);
    __builtin_amdgcn_sched_barrier(0);
    // S as fp16: the B fragments over the channels, and the chunk's incoming
    // state to the workspace (row 16 dt + r, columns 4 gq .. 4 gq + 3 of the tile)
    h4 Sq[NT_];
#pragma unroll
    for (int dt = 0; dt < NT_; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) Sq[dt][i] = static_cast<_Float16>(S[dt][i]);
    unsigned char* const so = stg[n & 1];
#pragma unroll
    for (int dt = 0; dt < NT_; ++dt) {
      const f4 tr = mma16(f4{0.f, 0.f, 0.f, 0.f}, Sq[dt], ident);
      h4 v;
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = static_cast<_Float16>(tr[i]);
      *reinterpret_cast<h4*>(so + ((16 * dt + r) * 32 + 16 * W + 4 * gq) * 2) = v;
    }
    h8 Sb[NJ];
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        Sb[j][i] = Sq[2 * j][i];
        Sb[j][4 + i] = Sq[2 * j + 1][i];
      }
    // v~ = U - W S, row tile ct
    f4 P[4];
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) P[ct] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) P[ct] = mma32(P[ct], AW[ct][j], Sb[j]);
    h8 AL[NT_][2];
#pragma unroll
    for (int dt = 0; dt < NT_; ++dt)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) AL[dt][kb] = frag(LY::NFW + 2 * dt + kb);
    f4 vt[4];
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) vt[ct] = Ut[ct] - P[ct];
    float* const vto = reinterpret_cast<float*>(so + LY::STG_VT);
#pragma unroll
    for (int ct = 0; ct < 4; ++ct)
#pragma unroll
      for (int i = 0; i < 4; ++i) vto[(16 * ct + 4 * gq + i) * 32 + 16 * W + r] = vt[ct][i];
    h8 Vb[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        Vb[kb][i] = static_cast<_Float16>(vt[2 * kb][i]);
        Vb[kb][4 + i] = static_cast<_Float16>(vt[2 * kb + 1][i]);
      }
    // S <- gamma_C S + (lambda k)^T v~, channel tile dt
#pragma unroll
    for (int dt = 0; dt < NT_; ++dt) {
      const f4 gc = *reinterpret_cast<const f4*>(cur + LY::OFF_GC + (16 * dt + 4 * gq) * 4);
      S[dt] = S[dt] * gc;
    }
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int dt = 0; dt < NT_; ++dt) S[dt] = mma32(S[dt], AL[dt][kb], Vb[kb]);
    lds_barrier();   // this buffer is free, the next one staged
  }
}

template <int D>
__global__ __launch_bounds__(64 * (2 + kFsProducers), 1) void kda_bwd_fscan16_kernel(BwdArgs a) {
  constexpr int NS = D / 32;
  __shared__ __attribute__((aligned(16))) unsigned char buf[2][FsLayout<D>::BYTES];
  __shared__ __attribute__((aligned(16))) unsigned char stg[2][FsLayout<D>::STG];
  int chain, split;
  if (!scan_slot<NS>(a.B * a.H, chain, split)) return;   // uniform per workgroup
  const int b = chain / a.H, h = chain - b * a.H;
  const int c0 = 32 * split;
  switch (threadIdx.x >> 6) {
    case 0: fs_chain<D, 0>(a, buf, stg, b, h, chain, c0); break;
    case 1: fs_chain<D, 1>(a, buf, stg, b, h, chain, c0); break;
    case 2: fs_producer<D, 0>(a, buf, stg, b, h, split); break;
    case 3: fs_producer<D, 1>(a, buf, stg, b, h, split); break;
    case 4: fs_producer<D, 2>(a, buf, stg, b, h, split); break;
    default: fs_producer<D, 3>(a, buf, stg, b, h, split); break;
  }
}

// A 16 x 16 accumulator tile (lane (r, gq): rows 4 gq + i, column r) into
// row-major hi / lo bf16 planes of pitch PB at (row0, col0): lanes r and r ^ 1
// swap one value of each row pair, so each lane writes packed column pairs
// (columns r & ~1, r | 1) of rows 4 gq + (r & 1) and 4 gq + 2 + (r & 1).
template <int PB>
__device__ __forceinline__ void acc_put_hl(const f4& v, int row0, int col0, __bf16* h, __bf16* l) {
  const int lane = threadIdx.x & 63, r = lane & 15, gq = lane >> 4;
  const bool odd = (r & 1) != 0;
  const float x0 = __shfl_xor(odd ? v[0] : v[1], 1, 64);
  const float x1 = __shfl_xor(odd ? v[2] : v[3], 1, 64);
  const int o = (row0 + 4 * gq + (odd ? 1 : 0)) * PB + col0 + (r & ~1);
  unsigned hh, ll;
  split2_bf16(odd ? x0 : v[0], odd ? v[1] : x0, hh, ll);
  *reinterpret_cast<unsigned*>(&h[o]) = hh;
  *reinterpret_cast<unsigned*>(&l[o]) = ll;
  split2_bf16(odd ? x1 : v[2], odd ? v[3] : x1, hh, ll);
  *reinterpret_cast<unsigned*>(&h[o + 2 * PB]) = hh;
  *reinterpret_cast<unsigned*>(&l[o + 2 * PB]) = ll;
}

// W of a chunk-head from its fp16 A fragments (rows x channels, the slot
// order of kda_internal.h) into hi / lo bf16 planes [64][PB] with the channel
// contiguous: each lane fragment is row 16 ct + r, channels 32 j + 4 gq .. + 3
// and 32 j + 16 + 4 gq .. + 3.
template <int D, int NTH>
struct WnTile {
  static constexpr int N = 4 * (D / 32) * 64;     // lane fragments
  static constexpr int PER = (N + NTH - 1) / NTH;
  static_assert(N % NTH == 0, "whole lane fragments per thread");
  uint4 w[PER];
  __device__ __forceinline__ void fetch(const void* src) {
#pragma unroll
    for (int p = 0; p < PER; ++p)
      w[p] = *reinterpret_cast<const uint4*>(static_cast<const u16*>(src) + (threadIdx.x + p * NTH) * 8);
  }
  template <int PB>
  __device__ __forceinline__ void put_hl(__bf16* h, __bf16* l) const {
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int e = threadIdx.x + p * NTH, f = e >> 6, ln = e & 63;
      const int ct = f / (D / 32), j = f - ct * (D / 32);
      const int row = 16 * ct + (ln & 15), ch0 = 32 * j + 4 * (ln >> 4);
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const f4 v = unpack4<2>(hf ? uint2{w[p].z, w[p].w} : uint2{w[p].x, w[p].y});
        uint2 hh, ll;
        split2_bf16(v[0], v[1], hh.x, ll.x);
        split2_bf16(v[2], v[3], hh.y, ll.y);
        *reinterpret_cast<uint2*>(&h[row * PB + ch0 + 16 * hf]) = hh;
        *reinterpret_cast<uint2*>(&l[row * PB + ch0 + 16 * hf]) = ll;
      }
    }
  }
};

// ---------------------------------------------------------------------------
// per chunk-head adjoint: one 512-thread workgroup per chunk-head, four
// phases separated by workgroup barriers, every phase in the same thread
// mapping so the partial dq, dk, dG stay in registers and each output is
// stored once:
//   1  dY = v~ dS'^T, dgq = do S^T, dW = dv~ S^T, dAqk = do v~^T (two
//      passes over the value channels); the epilogue forms dq's and dk's
//      terms and dG's first terms
//   2  Yw = T^T (-dW), Yu = T^T dv~; dv, dbeta's first terms, dk and dG
//   3  dL = -(Yw W^T + Yu U^T)
//   4  the score adjoints of the wave's row tile (row side) and key tile
//      (column side); dg's reverse cumsum; dq, dk, dg, dbeta stored
// ---------------------------------------------------------------------------
template <int D, int DTQ, int DTG, int DO>
__global__ __launch_bounds__(kChunkThreads) void kda_bwd_chunk_kernel(BwdArgs a) {
  typedef BwdDims<D> BD;
  constexpr int P = BD::P;
  constexpr int PC = kC + 4;          // [64][64] pitch: 16-byte aligned rows, row fragments conflict-free
  constexpr int NTH = kChunkThreads;
  constexpr int HW = 64;             // value columns per pass of phase 1
  constexpr int NH = D / HW;
  // LDS of the largest phase: phase 1's bf16 planes, phase 2's planes plus
  // the dk, dG hand-off and the row tiles' sums of g, phase 3's planes,
  // phase 4's dL, dAqk [64][PC] and q, k, G [64][P] plus beta
  constexpr int ACC0 = (2 * kC + 4 * D) * (kC + 8) / 2;   // floats of phase 2's bf16 planes
  constexpr int P4 = 2 * kC * PC + 3 * kC * P + kC + 17 * D + 40 * kC;   // floats of phase 4
  // [4][D] row tiles' sums of g, from phase 1's epilogue to phase 4: past
  // every buffer of phases 2 to 4
  constexpr int GS0 = cmax(ACC0 + 2 * kC * D, P4);
  constexpr int SMEM_FLOATS = cmax(cmax((6 * kC + 4 * D) * (HW + 8) / 2, GS0 + 4 * D), 8 * kC * (D + 8) / 2);
  __shared__ __attribute__((aligned(16))) float sm[SMEM_FLOATS];
  const int t = threadIdx.x;
  const int H = a.H;
  const int u = blockIdx.x / H, h = blockIdx.x - u * H;
  const ChunkRows cr = chunk_rows(a, u);
  const int64_t ch = static_cast<int64_t>(u) * H + h;
  auto in_idx = [&](int c, int d) { return ((cr.row0 + c) * H + h) * D + d; };
  // loads from pad rows (c >= len) read row 0 and are zeroed where used, so
  // no load sits inside a branch (whose end would wait for it)
  auto ld_q = [&](int c, int d) {
    const float x = ld1<DTQ>(a.q, in_idx(c < cr.len ? c : 0, d));
    return (c < cr.len) ? x * a.scale : 0.f;
  };
  auto ld_k = [&](int c, int d) {
    const float x = ld1<DTQ>(a.k, in_idx(c < cr.len ? c : 0, d));
    return (c < cr.len) ? x : 0.f;
  };
  auto ld_v = [&](int c, int d) {
    const float x = ld1<DTQ>(a.v, in_idx(c < cr.len ? c : 0, d));
    return (c < cr.len) ? x : 0.f;
  };
  auto ld_b = [&](int c) {
    const float x = ld1<DTG>(a.beta, (cr.row0 + (c < cr.len ? c : 0)) * H + h);
    return (c < cr.len) ? x : 0.f;
  };
  // Every phase works in one mapping: wave wv owns row tile mt = wv / 2 and
  // the NDT column tiles dt = (wv % 2) NDT + q of every [64][D] array (lane
  // (r, gq) holds rows 16 mt + 4 gq + i, column 16 dt + r), so the gradients
  // of q, k and G accumulate in registers from phase 1 to phase 4 and each
  // is stored once.  Phases 1-3 run on the matrix cores as bf16 hi / lo
  // triples.  Pad rows (c >= len) are never stored (their dG is zero: every
  // term carries a factor q_c or k_c).
  float* const gq_ = a.dq;
  float* const gk_ = a.dk;
  float* const gG_ = a.dg;
  float pq[D / 32][4], pk[D / 32][4], pG[D / 32][4];   // partial dq, dk, dG at this thread's positions
  constexpr int NDT = D / 32;          // column tiles per wave of a [64][D] product
  const int wv = t >> 6, l = t & 63, r16 = l & 15, gq = l >> 4;
  const int mt = wv >> 1, dg_ = wv & 1;
  const int mts = __builtin_amdgcn_readfirstlane(mt);   // mt as a wave-uniform (scalar) value

  float dbrD[4], dzp[NDT];             // dbeta partials (rows 16 mt + 4 gq + i), dz partials
#pragma unroll
  for (int i = 0; i < 4; ++i) dbrD[i] = 0.f;
#pragma unroll
  for (int q = 0; q < NDT; ++q) dzp[q] = 0.f;
  float dgc = 0.f;   // thread t < D: sum_n S[t][n] dS'[t][n]
  // G, k and q (times the scale; zero on pad rows) at this thread's positions
  // (rows 16 mt + 4 gq + i, columns 16 (dg_ NDT + q) + r16), read once in
  // phase 1's epilogue (G formed there from g): phase 2 shares the positions
  // and phase 4 takes its LDS copies of G, k, q from them
  // (q, k held as loaded: 16-bit inputs packed two to a register)
  typedef typename std::conditional<DTQ == 0, f4, uint2>::type H4;
  auto hload = [&](const void* src, int d) {   // rows 16 mt + 4 gq + i of column d (pad rows read row 0)
    H4 hv;
    if constexpr (DTQ == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int c = 16 * mt + 4 * gq + i;
        hv[i] = static_cast<const float*>(src)[in_idx(c < cr.len ? c : 0, d)];
      }
    } else {
      uint32_t b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int c = 16 * mt + 4 * gq + i;
        b[i] = static_cast<const u16*>(src)[in_idx(c < cr.len ? c : 0, d)];
      }
      hv.x = b[0] | (b[1] << 16);
      hv.y = b[2] | (b[3] << 16);
    }
    return hv;
  };
  auto hget = [&](const H4& hv, int i) {   // element i, zero on pad rows
    float x;
    if constexpr (DTQ == 0) x = hv[i];
    else {
      const uint32_t w = (i < 2) ? hv.x : hv.y;
      const u16 bits = static_cast<u16>((i & 1) ? (w >> 16) : (w & 0xFFFFu));
      x = (DTQ == 1) ? bf16_to_f32(bits) : f16bits_to_f32(bits);
    }
    return (16 * mt + 4 * gq + i < cr.len) ? x : 0.f;
  };
  float gH[NDT][4], gLast[NDT];
  H4 kH[NDT], qH[NDT];
  constexpr int EF = BwdWs<DTQ != 0>::F;    // S_in, T, W

  // Phase 1's dk and dG terms reach phase 2 (same thread, same positions)
  // through LDS past phase 2's buffers, not through dk and dg in memory.
  float* const sAcc = sm + ACC0;   // [2][64][D]: dk, dG
  static_assert(ACC0 + 2 * kC * D <= SMEM_FLOATS, "phase 1 -> 2 accumulators");

  // ---- phase 1: dY = v~ dS'^T, dgq = do S^T, dW = -dv~ S^T, dAqk = do v~^T
  // (K = dv in passes of HW)
  // The operands go to LDS as hi / lo bf16 planes (K contiguous) and each
  // product runs as three bf16 MFMAs per 32-wide K block (hi hi + hi lo +
  // lo hi, about 2^-16 of each product dropped); dW accumulates +dv~ S^T and
  // is negated where phase 2 takes it.
  f4 dW[NDT];
  // dAqk = tril(do v~^T), two 16 x 16 tiles per wave (row tile mt, key tiles
  // 2 (wv % 2) + q), from phase 1's do and v~ planes: K = the value channels
  // of each pass; key tiles above the row tile are skipped (masked in phase 3)
  f4 dAa[2];
  const int kt0 = 2 * (wv & 1);
  const bool live0 = kt0 <= mts, live1 = kt0 + 1 <= mts;   // wave-uniform
#pragma unroll
  for (int q = 0; q < 2; ++q) dAa[q] = f4{0.f, 0.f, 0.f, 0.f};
  TTile<kC, NTH, EF> tT;     // phase 2's T, loaded during phase 1's last pass
  // dv~ in row pairs: column block hp is phase 1's pass hp operand, and the
  // whole tile phase 2's dv~^T (one read of dv~ serves both)
  TTile<D, NTH> tY;
  static_assert(TTile<D, NTH>::PER == D / 64 && TTile<D, NTH>::G * 4 == 64, "one column block per pass");
  {
    f4 dY[NDT], dgq[NDT];
#pragma unroll
    for (int q = 0; q < NDT; ++q)
#pragma unroll
      for (int i = 0; i < 4; ++i) dY[q][i] = dgq[q][i] = dW[q][i] = 0.f;
    constexpr int PB = HW + 8;         // bf16 pitch: rows of 32-wide K blocks start 16-byte aligned
    static_assert((6 * kC + 4 * D) * PB / 2 <= SMEM_FLOATS, "phase 1 LDS");
    __bf16* const sVh = reinterpret_cast<__bf16*>(sm);
    __bf16* const sVl = sVh + kC * PB;
    __bf16* const sOh = sVl + kC * PB;
    __bf16* const sOl = sOh + kC * PB;
    __bf16* const sUh = sOl + kC * PB;   // dv~
    __bf16* const sUl = sUh + kC * PB;
    __bf16* const sSh = sUl + kC * PB;
    __bf16* const sSl = sSh + D * PB;
    __bf16* const sDh = sSl + D * PB;    // dS'
    __bf16* const sDl = sDh + D * PB;
    // a pass's operands are loaded during the previous pass's products
    Tile<kC, HW, NTH> pV;
    Tile<D, HW, NTH, EF> pS;
    Tile<D, HW, NTH> pDS;
    InTile<DO, D, HW, NTH> pDo;
    auto fetch_pass = [&](int hp) {
      const int n0 = HW * hp;
      pV.fetch(a.VT + ch * kC * D, D, n0);
      tY.fetch_block(a.DVT + ch * kC * D, D, 0, hp);
      pS.fetch(ws_at<EF>(a.SI, ch * D * D), D, n0);
      pDS.fetch(a.DS + ch * D * D, D, n0);
      pDo.fetch(a.dout, cr.row0, cr.len, H, h, n0);
    };
    fetch_pass(0);
#pragma unroll
    for (int hp = 0; hp < NH; ++hp) {
      put_hl<PB>(pV, sVh, sVl);
      tY.template put_rows_hl<PB>(hp, sUh, sUl);
      put_hl<PB>(pS, sSh, sSl);
      put_hl<PB>(pDS, sDh, sDl);
      put_hl<PB>(pDo, sOh, sOl);
      __syncthreads();
      if (hp + 1 < NH) fetch_pass(hp + 1);
      else tT.fetch(ws_at<EF>(a.TM, ch * kC * kC), kC, 0);   // phase 2's T
#pragma unroll
      for (int kb = 0; kb < HW / 32; ++kb) {
        const int ka = (16 * mt + r16) * PB + 32 * kb + 8 * gq;
        const b8 vh = *reinterpret_cast<const b8*>(&sVh[ka]), vl = *reinterpret_cast<const b8*>(&sVl[ka]);
        const b8 oh = *reinterpret_cast<const b8*>(&sOh[ka]), ol = *reinterpret_cast<const b8*>(&sOl[ka]);
        const b8 uh = *reinterpret_cast<const b8*>(&sUh[ka]), ul = *reinterpret_cast<const b8*>(&sUl[ka]);
#pragma unroll
        for (int q = 0; q < NDT; ++q) {
          const int kbb = (16 * (dg_ * NDT + q) + r16) * PB + 32 * kb + 8 * gq;
          const b8 sh = *reinterpret_cast<const b8*>(&sSh[kbb]), sl = *reinterpret_cast<const b8*>(&sSl[kbb]);
          const b8 dh = *reinterpret_cast<const b8*>(&sDh[kbb]), dl = *reinterpret_cast<const b8*>(&sDl[kbb]);
          dY[q] = mma3_bf16(dY[q], vh, vl, dh, dl);
          dgq[q] = mma3_bf16(dgq[q], oh, ol, sh, sl);
          dW[q] = mma3_bf16(dW[q], uh, ul, sh, sl);
        }
        if (live0) {
#pragma unroll
          for (int q = 0; q < 2; ++q) {
            if (q == 1 && !live1) continue;
            const int kv = (16 * (kt0 + q) + r16) * PB + 32 * kb + 8 * gq;
            dAa[q] = mma3_bf16(dAa[q], oh, ol, *reinterpret_cast<const b8*>(&sVh[kv]),
                               *reinterpret_cast<const b8*>(&sVl[kv]));
          }
        }
      }
      if (t < D) {
#pragma unroll 2
        for (int n8 = 0; n8 < HW; n8 += 8) {
          const b8 sh = *reinterpret_cast<const b8*>(&sSh[t * PB + n8]), sl = *reinterpret_cast<const b8*>(&sSl[t * PB + n8]);
          const b8 dh = *reinterpret_cast<const b8*>(&sDh[t * PB + n8]), dl = *reinterpret_cast<const b8*>(&sDl[t * PB + n8]);
#pragma unroll
          for (int e = 0; e < 8; ++e)
            dgc = fmaf(static_cast<float>(sh[e]) + static_cast<float>(sl[e]),
                       static_cast<float>(dh[e]) + static_cast<float>(dl[e]), dgc);
        }
      }
      __syncthreads();
    }
    // G_c = log2(e) sum_{c' <= c} g_c' at this thread's positions, from g:
    // the prefix over the lane's four rows, plus the lane groups above it in
    // the row tile (shuffles), plus the row tiles above (their sums through
    // LDS, past phase 2's buffers).  G_{C-1} sums the four tile sums in the
    // order the last row's prefix does, so the two agree bit for bit.
    float* const sGs = sm + GS0;
#pragma unroll
    for (int q = 0; q < NDT; ++q) {
      const int d = 16 * (dg_ * NDT + q) + r16;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int c = 16 * mt + 4 * gq + i;
        const float x = ld1<DTG>(a.g, in_idx(c < cr.len ? c : 0, d));
        gH[q][i] = (c < cr.len) ? x : 0.f;
      }
      qH[q] = hload(a.q, d);
      kH[q] = hload(a.k, d);
    }
#pragma unroll
    for (int q = 0; q < NDT; ++q) {
#pragma unroll
      for (int i = 1; i < 4; ++i) gH[q][i] += gH[q][i - 1];
      const float tot = gH[q][3];
      const float t1 = __shfl_up(tot, 16), t2 = __shfl_up(tot, 32), t3 = __shfl_up(tot, 48);
      const float ex = (gq >= 1 ? t1 : 0.f) + (gq >= 2 ? t2 : 0.f) + (gq >= 3 ? t3 : 0.f);
#pragma unroll
      for (int i = 0; i < 4; ++i) gH[q][i] += ex;
      if (gq == 3) sGs[mt * D + 16 * (dg_ * NDT + q) + r16] = gH[q][3];
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < NDT; ++q) {
      const int d = 16 * (dg_ * NDT + q) + r16;
      float pre = 0.f, run = 0.f;
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        if (m == mts) pre = run;
        run += sGs[m * D + d];
      }
      gLast[q] = run * kLog2e;
#pragma unroll
      for (int i = 0; i < 4; ++i) gH[q][i] = (gH[q][i] + pre) * kLog2e;
    }
    // dq = dgq gamma; dG = dgq q gamma - dY k lambda; dk = dY lambda
#pragma unroll
    for (int q = 0; q < NDT; ++q) {
      const int d = 16 * (dg_ * NDT + q) + r16;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int c = 16 * mt + 4 * gq + i;
        const float gam = ex2(gH[q][i]), lam = ex2(gLast[q] - gH[q][i]);
        const float dz = dY[q][i] * hget(kH[q], i) * lam;
        dzp[q] += dz;
        pq[q][i] = dgq[q][i] * gam * a.scale;
        sAcc[c * D + d] = dY[q][i] * lam;
        sAcc[(kC + c) * D + d] = dgq[q][i] * (hget(qH[q], i) * a.scale) * gam - dz;
      }
    }
  }

  // ---- phase 2: Yw = T^T dW, Yu = T^T dv~ (K = the chunk's 64 rows), as
  // bf16 hi / lo triples: T^T, (-dW)^T and dv~^T in LDS with the chunk row
  // contiguous; T[c][m] is zero for c < m, so row tile mt starts at the
  // K block holding row 16 mt.
  f4 Yw[NDT], Yu[NDT];
  // W from its row-major array (fp32 inputs) or its fp16 A fragments (16-bit)
  typename std::conditional<EF == 0, Tile<kC, D, NTH>, WnTile<D, NTH>>::type tW3;
  Tile<kC, D, NTH> tU3;
  {
    constexpr int PB = kC + 8;
    static_assert((2 * kC + 4 * D) * PB / 2 <= ACC0, "phase 2 planes end below sAcc");
    __bf16* const sTh = reinterpret_cast<__bf16*>(sm);   // T^T [64][64]
    __bf16* const sTl = sTh + kC * PB;
    __bf16* const sXh = sTl + kC * PB;                   // (-dW)^T [D][64]
    __bf16* const sXl = sXh + D * PB;
    __bf16* const sYh = sXl + D * PB;                    // dv~^T [D][64]
    __bf16* const sYl = sYh + D * PB;
#pragma unroll
    for (int q = 0; q < NDT; ++q) {
      const int o = (16 * (dg_ * NDT + q) + r16) * PB + 16 * mt + 4 * gq;
      uint2 hh, ll;
      split2_bf16(-dW[q][0], -dW[q][1], hh.x, ll.x);
      split2_bf16(-dW[q][2], -dW[q][3], hh.y, ll.y);
      *reinterpret_cast<uint2*>(&sXh[o]) = hh;
      *reinterpret_cast<uint2*>(&sXl[o]) = ll;
    }
    tT.template put_hl<PB>(sTh, sTl);
    tY.template put_hl<PB>(sYh, sYl);
    __syncthreads();
    H4 vH[NDT];   // the epilogue's v and beta, during the products
    float bH[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) bH[i] = ld_b(16 * mt + 4 * gq + i);
#pragma unroll
    for (int q = 0; q < NDT; ++q) vH[q] = hload(a.v, 16 * (dg_ * NDT + q) + r16);
#pragma unroll
    for (int q = 0; q < NDT; ++q)
#pragma unroll
      for (int i = 0; i < 4; ++i) Yw[q][i] = Yu[q][i] = 0.f;
    for (int kb = mts >> 1; kb < kC / 32; ++kb) {
      const int ka = (16 * mt + r16) * PB + 32 * kb + 8 * gq;
      const b8 th = *reinterpret_cast<const b8*>(&sTh[ka]), tl = *reinterpret_cast<const b8*>(&sTl[ka]);
#pragma unroll
      for (int q = 0; q < NDT; ++q) {
        const int kbb = (16 * (dg_ * NDT + q) + r16) * PB + 32 * kb + 8 * gq;
        Yw[q] = mma3_bf16(Yw[q], th, tl, *reinterpret_cast<const b8*>(&sXh[kbb]),
                          *reinterpret_cast<const b8*>(&sXl[kbb]));
        Yu[q] = mma3_bf16(Yu[q], th, tl, *reinterpret_cast<const b8*>(&sYh[kbb]),
                          *reinterpret_cast<const b8*>(&sYl[kbb]));
      }
    }
    __syncthreads();
    // dG += Yw k beta gamma; dk += Yw gamma beta; dv = Yu beta; dbeta += Yw gamma k + Yu v
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = 16 * mt + 4 * gq + i;
      const bool live = c < cr.len;
      const float bc = bH[i];
      float kv[NDT], vv[NDT], oG[NDT], ok[NDT];
#pragma unroll
      for (int q = 0; q < NDT; ++q) {
        const int d = 16 * (dg_ * NDT + q) + r16;
        kv[q] = hget(kH[q], i);
        vv[q] = hget(vH[q], i);
        oG[q] = sAcc[(kC + c) * D + d];
        ok[q] = sAcc[c * D + d];
      }
#pragma unroll
      for (int q = 0; q < NDT; ++q) {
        const int d = 16 * (dg_ * NDT + q) + r16;
        const float gam = ex2(gH[q][i]);
        dbrD[i] += Yw[q][i] * gam * kv[q] + Yu[q][i] * vv[q];
        pG[q][i] = oG[q] + Yw[q][i] * kv[q] * bc * gam;
        pk[q][i] = ok[q] + Yw[q][i] * gam * bc;
        if (live) a.dv[in_idx(c, d)] = Yu[q][i] * bc;
      }
    }
    __syncthreads();   // sAcc read before phase 3's operands overwrite it
  }

  // ---- phase 3: dL = strict(-(Yw W^T + Yu U^T)) [64][64] (dAqk came from
  // phase 1), two 16 x 16 tiles per wave: row tile mt, key tiles 2 (wv % 2) + q,
  // as bf16 hi / lo triples (operands row-major with the channel, the K index,
  // contiguous); key tiles above the row tile are masked to zero and skipped.
  float* const sDL = sm;                 // phase 4's operands, written at the end of phase 3
  float* const sDA = sDL + kC * PC;
  // past phase 4's dL, dAqk, q, k, G, beta: [16][D] dz partials, then the
  // per-column base of dg [D]
  float* const sRed4 = sm + 2 * kC * PC + 3 * kC * P + kC;
  float* const sBase = sRed4 + 16 * D;
  // then the row partial sums of dbeta: [64][32] from phase 2 (written at the
  // start of phase 3, past its planes), [64][8] from phase 4 (per column tile)
  float* const sDbD = sBase + D;
  float* const sDb4 = sDbD + kC * 32;
  static_assert(P4 <= GS0 && GS0 + 4 * D <= SMEM_FLOATS, "phase 4 LDS, below the sums of g");
  static_assert(8 * kC * (D + 8) / 2 <= 2 * kC * PC + 3 * kC * P + kC + 17 * D, "phase 3 planes end below sDbD");
  {
    constexpr int PB = D + 8;            // bf16 pitch: 16-byte aligned K blocks, rows 4 banks apart
    static_assert(8 * kC * PB / 2 <= SMEM_FLOATS, "phase 3 LDS");
    __bf16* const sAh = reinterpret_cast<__bf16*>(sm);   // Yw
    __bf16* const sAl = sAh + kC * PB;
    __bf16* const sBh = sAl + kC * PB;                   // Yu
    __bf16* const sBl = sBh + kC * PB;
    __bf16* const sWh = sBl + kC * PB;
    __bf16* const sWl = sWh + kC * PB;
    __bf16* const sUh = sWl + kC * PB;
    __bf16* const sUl = sUh + kC * PB;
#pragma unroll
    for (int q = 0; q < NDT; ++q) {
      acc_put_hl<PB>(Yw[q], 16 * mt, 16 * (dg_ * NDT + q), sAh, sAl);
      acc_put_hl<PB>(Yu[q], 16 * mt, 16 * (dg_ * NDT + q), sBh, sBl);
    }
    if constexpr (EF == 0) tW3.fetch(a.WM + ch * kC * D, D, 0);
    else tW3.fetch(static_cast<const u16*>(a.FWN) + ch * kC * D);
    tU3.fetch(a.UM + ch * kC * D, D, 0);
    if constexpr (EF == 0) put_hl<PB>(tW3, sWh, sWl);
    else tW3.template put_hl<PB>(sWh, sWl);
    put_hl<PB>(tU3, sUh, sUl);
#pragma unroll
    for (int i = 0; i < 4; ++i) sDbD[(16 * mt + 4 * gq + i) * 32 + 16 * dg_ + r16] = dbrD[i];
    __syncthreads();
    f4 dLa[2];
#pragma unroll
    for (int q = 0; q < 2; ++q) dLa[q] = f4{0.f, 0.f, 0.f, 0.f};
    if (live0) {
#pragma unroll 2
      for (int kb = 0; kb < D / 32; ++kb) {
        const int ka = (16 * mt + r16) * PB + 32 * kb + 8 * gq;
        const b8 ywh = *reinterpret_cast<const b8*>(&sAh[ka]), ywl = *reinterpret_cast<const b8*>(&sAl[ka]);
        const b8 yuh = *reinterpret_cast<const b8*>(&sBh[ka]), yul = *reinterpret_cast<const b8*>(&sBl[ka]);
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          if (q == 1 && !live1) continue;
          const int kbb = (16 * (kt0 + q) + r16) * PB + 32 * kb + 8 * gq;
          dLa[q] = mma3_bf16(dLa[q], ywh, ywl, *reinterpret_cast<const b8*>(&sWh[kbb]),
                             *reinterpret_cast<const b8*>(&sWl[kbb]));
          dLa[q] = mma3_bf16(dLa[q], yuh, yul, *reinterpret_cast<const b8*>(&sUh[kbb]),
                             *reinterpret_cast<const b8*>(&sUl[kbb]));
        }
      }
    }
    __syncthreads();   // every read of the planes done before sDL, sDA overwrite them
    // phase 4's masked operands
#pragma unroll
    for (int q = 0; q < 2; ++q)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int c = 16 * mt + 4 * gq + i, ii = 16 * (2 * dg_ + q) + r16;
        sDL[c * PC + ii] = (ii < c) ? -dLa[q][i] : 0.f;
        sDA[c * PC + ii] = (ii <= c) ? dAa[q][i] : 0.f;
      }
    // dz column partials (slot 4 mt + gq) for the per-column base of dg
#pragma unroll
    for (int q = 0; q < NDT; ++q) sRed4[(4 * mt + gq) * D + 16 * (dg_ * NDT + q) + r16] = dzp[q];
    __syncthreads();
  }

  // ---- phase 4: score adjoints.  With dA = sDA, dL = sDL (masked):
  //   row side  rA[c] = sum_i dA[c][i] k_i 2^(G_c - G_i),  rK likewise with dL;
  //   col side  cS[i] = sum_c (dA[c][i] q_c + dL[c][i] beta_c k_c) 2^(G_c - G_i);
  //   dq += rA; dk += rK beta + cS; dG += rA q + rK k beta - cS k; dbeta_c += sum_d rK k_c
  // (q carries the scale).  Off-diagonal tile pairs (row tile R > key tile s)
  // factor the decay at the row tile's first row a, 2^(G_c - G_a) 2^(G_a - G_i),
  // both <= 1, and run on the matrix cores: (16 x 16 block) x (k_i 2^(G_a - G_i))
  // for the row side, (block)^T x (q_c 2^(G_c - G_a)) for the column side.
  // Diagonal tiles are anchored the same way (their key factors >= 1, bounded
  // by the tile's decay) unless the tile decays past 2^-kDiagAnchorLog2 in a
  // column of the wave; those take 2^-|G_c - G_i| per element.  Wave (mt, half)
  // forms, for each of its column tiles, the row side of row tile mt (key
  // tiles s <= mt) and the column side of key tile mt (row tiles R >= mt), so
  // the results land on the positions whose partial sums it holds.
  constexpr int NCT = D / 16;
  {
    float* sQ = sDA + kC * PC;       // q * scale
    float* sK = sQ + kC * P;
    float* sG = sK + kC * P;
    float* sB = sG + kC * P;
#pragma unroll
    for (int q = 0; q < NDT; ++q)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int o = (16 * mt + 4 * gq + i) * P + 16 * (dg_ * NDT + q) + r16;
        sQ[o] = hget(qH[q], i) * a.scale;
        sK[o] = hget(kH[q], i);
        sG[o] = gH[q][i];
      }
    if (t < kC) sB[t] = ld_b(t);
    if (t < D) {   // dg[c] = base + sum_{c' >= c} dG[c']: the G_C terms and the dz terms
      const float* sGs = sm + GS0;   // G_{C-1} of column t, summed as in phase 1's epilogue
      float acc = dgc * ex2((((sGs[t] + sGs[D + t]) + sGs[2 * D + t]) + sGs[3 * D + t]) * kLog2e);
      for (int r = 0; r < 16; ++r) acc += sRed4[r * D + t];
      sBase[t] = acc;
    }
    __syncthreads();
    float* const sTile = sRed4;      // [4][D] dG column sums of each row tile (sRed4 is read above)
    const int a0 = 16 * mt;
    float sfx[NDT][4], abv[NDT];
#pragma unroll
    for (int q = 0; q < NDT; ++q) {
      const int d = 16 * (dg_ * NDT + q) + r16;
      const float ga = sG[a0 * P + d];
      f4 accA = {0.f, 0.f, 0.f, 0.f}, accK = {0.f, 0.f, 0.f, 0.f};
      // row side: key tiles below the row tile
      for (int sk = 0; sk < mts; ++sk) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int i = 16 * sk + 4 * k + gq;
          const float kb = sK[i * P + d] * ex2(ga - sG[i * P + d]);   // k_i 2^(G_a - G_i)
          accA = mfma4(sDA[(a0 + r16) * PC + 16 * sk + 4 * k + gq], kb, accA);
          accK = mfma4(sDL[(a0 + r16) * PC + 16 * sk + 4 * k + gq], kb, accK);
        }
      }
      // column side: row tiles above the key tile, the furthest first
      float colS[4] = {0.f, 0.f, 0.f, 0.f};
      for (int R = 3; R > mts; --R) {
        const int aR = 16 * R;
        const float gR = sG[aR * P + d];
        f4 cS = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int c = aR + 4 * k + gq;
          const float fr = ex2(sG[c * P + d] - gR);   // q_c 2^(G_c - G_R), beta_c k_c 2^(G_c - G_R)
          cS = mfma4(sDA[c * PC + a0 + r16], sQ[c * P + d] * fr, cS);
          cS = mfma4(sDL[c * PC + a0 + r16], sK[c * P + d] * sB[c] * fr, cS);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) colS[e] += cS[e] * ex2(gR - sG[(a0 + 4 * gq + e) * P + d]);
      }
      float gc[4], rA[4], rK[4], cS[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        gc[e] = sG[(a0 + 4 * gq + e) * P + d];
        rA[e] = rK[e] = cS[e] = 0.f;
      }
      // The diagonal tile on the matrix cores, anchored at its first row a
      // like the off-diagonal ones: row side (block) x (k_y 2^(G_a - G_y)),
      // column side (block)^T x (q_c 2^(G_c - G_a)), times 2^(G_c - G_a) and
      // 2^(G_a - G_i) afterwards.  Key factors here are >= 1, up to the
      // tile's decay in the column; the masked cotangents zero every pair
      // whose factor would exceed 1 overall.  A tile that decays by more
      // than 2^-kDiagAnchorLog2 in one of the wave's columns (the factors
      // would leave fp32 headroom for the cotangents) takes the per-element
      // form below.
      if (!__any(ga - sG[(a0 + 15) * P + d] > kDiagAnchorLog2)) {
        f4 cd = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int y = a0 + 4 * k + gq;
          const float fr = ex2(sG[y * P + d] - ga);
          const float kb = sK[y * P + d] * ex2(ga - sG[y * P + d]);   // k_y 2^(G_a - G_y)
          accA = mfma4(sDA[(a0 + r16) * PC + y], kb, accA);
          accK = mfma4(sDL[(a0 + r16) * PC + y], kb, accK);
          cd = mfma4(sDA[y * PC + a0 + r16], sQ[y * P + d] * fr, cd);
          cd = mfma4(sDL[y * PC + a0 + r16], sK[y * P + d] * sB[y] * fr, cd);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) cS[e] = cd[e] * ex2(ga - gc[e]);
      } else {
        // With G non-increasing (g <= 0), the pair (c, a0 + y) of the row
        // side (y <= x) decays by 2^(G_c - G_y) and the pair (a0 + y, c) of
        // the column side (y >= x) by 2^(G_y - G_c): both are 2^-|G_c - G_y|,
        // and the masked cotangents zero the side a given y does not belong to.
        // Row y's G, k, q, beta are read once for the lane's four rows c.
#pragma unroll 1
        for (int y4 = 0; y4 < 16; y4 += 4) {
          f4 rowA[4], rowL[4];   // dA[c][a0 + y4 .. + 3], dL likewise, for the lane's rows c
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int c = a0 + 4 * gq + e;
            rowA[e] = *reinterpret_cast<const f4*>(&sDA[c * PC + a0 + y4]);
            rowL[e] = *reinterpret_cast<const f4*>(&sDL[c * PC + a0 + y4]);
          }
#pragma unroll
          for (int yy = 0; yy < 4; ++yy) {
            const int y = y4 + yy;
            const float gy = sG[(a0 + y) * P + d], ky = sK[(a0 + y) * P + d];
            const float qy = sQ[(a0 + y) * P + d], by = sB[a0 + y];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int c = a0 + 4 * gq + e;
              const float ev = ex2(-fabsf(gc[e] - gy));
              const float kr = ky * ev;
              rA[e] = fmaf(rowA[e][yy], kr, rA[e]);
              rK[e] = fmaf(rowL[e][yy], kr, rK[e]);
              cS[e] = fmaf(sDA[(a0 + y) * PC + c], qy * ev, cS[e]);
              cS[e] = fmaf(sDL[(a0 + y) * PC + c], by * kr, cS[e]);
            }
          }
        }
      }
      float gn[4], dbq[4];   // this tile's dG (zero on pad rows), dbeta terms
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int c = a0 + 4 * gq + e;
        const float kc = sK[c * P + d], qc = sQ[c * P + d], bc = sB[c];
        const float f = ex2(gc[e] - ga);   // accA, accK: every tile pair but a per-element diagonal
        rA[e] = fmaf(accA[e], f, rA[e]);
        rK[e] = fmaf(accK[e], f, rK[e]);
        if (mts < 3) cS[e] += colS[e];
        dbq[e] = rK[e] * kc;
        gn[e] = (c < cr.len) ? pG[q][e] + rA[e] * qc + rK[e] * kc * bc - cS[e] * kc : 0.f;
        if (c < cr.len) {
          const int64_t o = in_idx(c, d);
          gq_[o] = pq[q][e] + rA[e] * a.scale;
          gk_[o] = pk[q][e] + rK[e] * bc + cS[e];
        }
      }
      // reverse cumsum down the column: within the lane's four rows, then
      // over the row groups gq' > gq of the tile (lanes 16 gq' + r16); the
      // tiles below come after the barrier
      sfx[q][3] = gn[3];
      sfx[q][2] = gn[2] + sfx[q][3];
      sfx[q][1] = gn[1] + sfx[q][2];
      sfx[q][0] = gn[0] + sfx[q][1];
      const float x1 = __shfl_down(sfx[q][0], 16, 64), x2 = __shfl_down(sfx[q][0], 32, 64);
      const float x3 = __shfl_down(sfx[q][0], 48, 64);
      abv[q] = (gq < 3 ? x1 : 0.f) + (gq < 2 ? x2 : 0.f) + (gq < 1 ? x3 : 0.f);
      if (gq == 0) sTile[mt * D + d] = sfx[q][0] + abv[q];   // the tile's column sum
      // dbeta partials: sum over the 16 columns of the tile
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float v = dbq[e];
#pragma unroll
        for (int off = 8; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
        if (r16 == 0) sDb4[(a0 + 4 * gq + e) * 8 + dg_ * NDT + q] = v;
      }
    }
    __syncthreads();   // phase 4's LDS reads done; every tile's column sums written
#pragma unroll
    for (int q = 0; q < NDT; ++q) {
      const int d = 16 * (dg_ * NDT + q) + r16;
      float carry = 0.f;   // the tiles below, the furthest first
      for (int R = 3; R > mts; --R) carry += sTile[R * D + d];
      const float base = sBase[d] + carry + abv[q];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int c = a0 + 4 * gq + e;
        if (c < cr.len) gG_[in_idx(c, d)] = base + sfx[q][e];
      }
    }
  }

  // ---- outputs: dbeta (its row partial sums in LDS before phase 4's last barrier)
  {
    if (t < kC && t < cr.len) {
      float acc = 0.f;
      for (int j = 0; j < NCT; ++j) acc += sDb4[t * 8 + j];
      for (int j = 0; j < 32; ++j) acc += sDbD[t * 32 + j];
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
  if constexpr (DTQ != 0)
    hipLaunchKernelGGL((kda_bwd_fscan16_kernel<D>), dim3(scan_grid), dim3(64 * (2 + kFsProducers)), 0, s, a);
  else
    hipLaunchKernelGGL((kda_bwd_fscan_kernel<D, false>), dim3(scan_grid), dim3(ScanThreads<D>::value), 0, s, a);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  if constexpr (DTQ != 0)
    hipLaunchKernelGGL((kda_bwd_rscan16_kernel<D, DO>), dim3(scan_grid), dim3(64 * (2 + kRsProducers)), 0, s, a);
  else
    hipLaunchKernelGGL((kda_bwd_rscan_kernel<D, DO, false>), dim3(scan_grid), dim3(ScanThreads<D>::value), 0, s, a);
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
