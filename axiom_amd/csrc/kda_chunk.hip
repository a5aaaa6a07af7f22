// Chunked KDA forward in WY/UT form for gfx950 (CDNA4).
//
// Math (per head, chunk length C = 64, g = log alpha <= 0 per channel,
// G = inclusive cumsum of g inside the chunk, gamma = exp(G)), restating
// net/kda.py:669-702 (cc_chunk_step) of the reference:
//   Aqk[c,i] = sum_d q[c,d] k[i,d] exp(G[c,d]-G[i,d])          (c >= i)
//   L[c,i]   = beta_c sum_d k[c,d] k[i,d] exp(G[c,d]-G[i,d])   (c >  i)
//   T = (I+L)^-1,  W = T (beta gamma k),  U = T (beta v)
//   v~ = U - W S,  o = (gamma q) S + Aqk v~,
//   S' = diag(gamma_C) S + (lambda k)^T v~,  lambda = exp(G_C - G)
//
// Decay factors.  The chunk is cut into four 16-row tiles.  With Gt the
// tile-local inclusive cumsum (log2 units) and D the tile total, every lane
// needs only R = 2^Gt (<= 1) and Cf = 2^(D - Gt) (<= 1):
//   off-diagonal tile pair (r > s):  2^(G_c - G_i) = R_c * M_rs * Cf_i,
//     M_rs = 2^(sum of the totals of the tiles strictly between) <= 1,
//     so both MFMA operands stay in [0, 1] and run in fp16;
//   diagonal tile (c >= i):  2^(G_c - G_i) = (R_c 2^-D) * Cf_i, operands up
//     to 2^|D|: on fp16 MFMA when the tile's operands stay below 2^15 (tile
//     decay above 2^-12, |k Cf|, |k R|, |q R| <= 8), else on the bf16 MFMA
//     as a three-product hi/lo split (fp32 range, ~16 significant bits),
//     and on fp32 MFMA (16x16x4) in exact mode; a tile whose total decay
//     passes 2^-100 takes a slower path that splits each pair at the highest
//     bit where c and i differ, through an anchor row between them, so every
//     factor stays <= 1 however strong the decay;
//   gamma = R * 2^(totals before the tile), lambda = Cf * 2^(totals after).
// The per-channel constants (2^pre, 2^post, 2^-D, M) are computed once per
// wave into LDS.
//
// Work split: wave w of a 256-thread workgroup owns rows 16w..16w+15 (its
// code is compiled per w so tile-dependent loops are static), lane
// (r = l & 15, gq = l >> 4) owns row 16w + r and the 8 channel slots of lane
// group gq in every 32-wide K step (see kda_common.h).
//
// Kernels:
//  * kda_intra_kernel -- one workgroup per chunk-head; writes W, U, Aqk,
//    gamma*q, lambda*k and gamma_C to the workspace in MFMA fragment order.
//  * kda_state_col_kernel (16-bit inputs) -- one workgroup per (chain,
//    32-column dv slice): two compute waves hold the fp32 state slice in MFMA
//    accumulators and walk the chain's chunks while four producer waves copy
//    each chunk's operands into LDS two chunks ahead and store o.
//  * kda_state_wide_kernel (16-bit inputs, >= 256 chains) -- the same with one
//    workgroup per whole chain.
//  * kda_overlap_kernel (16-bit inputs, <= 24 chains) -- one segment's
//    state-slice workgroups and the next segment's intra work in one launch.
//  * kda_state_kernel (exact mode, fp32 inputs) -- one workgroup per (chain,
//    32-column dv slice) with fp32 operands.

#include <type_traits>

#include "kda_common.h"
#include "kda_internal.h"

namespace kda {

constexpr int kC = 64;

// ----------------------------------------------------------------------------
// non-finite detection of the results (fp16 operand range)
//
// Each lane keeps the sum of the magnitudes of the values it stores: an inf
// or NaN among them makes the sum non-finite, and one add per value (with
// the |x| source modifier) is all the checking the store paths pay.  Inside
// the supported operand range a sum of finite values stays far below fp32's
// limit (|o| < 2^23 per element for unit-norm q, k; a lane stores a few
// values per chunk).
// ----------------------------------------------------------------------------
__device__ __forceinline__ float abs_sum_f32x4(const uint4 v) {
  return (fabsf(__uint_as_float(v.x)) + fabsf(__uint_as_float(v.y))) +
         (fabsf(__uint_as_float(v.z)) + fabsf(__uint_as_float(v.w)));
}
__device__ __forceinline__ float abs_sum_bf16x2(const uint32_t w) {
  return fabsf(__uint_as_float(w << 16)) + fabsf(__uint_as_float(w & 0xFFFF0000u));
}
__device__ __forceinline__ float abs_sum_bf16x8(const uint4 v) {
  return (abs_sum_bf16x2(v.x) + abs_sum_bf16x2(v.y)) + (abs_sum_bf16x2(v.z) + abs_sum_bf16x2(v.w));
}
// sets the call's status bit from one lane when any lane of the wave holds a
// non-finite magnitude sum
__device__ __forceinline__ void report_nonfinite(int* status, float mag) {
  const bool bad = !(mag <= 3.402823466e38f);   // inf or NaN
  if (status != nullptr && __any(bad) && (threadIdx.x & 63) == 0) atomicOr(status, kStatusNonFinite);
}

// ----------------------------------------------------------------------------
// chunk-unit geometry
// ----------------------------------------------------------------------------
struct UnitRef {
  int seq;        // sequence (dense: batch index)
  int n;          // chunk index inside the sequence
  int64_t row0;   // first token (global token index into [B*T] or the packed T)
  int len;        // valid rows, 1..64
};

// u: the launch's unit (its workspace slot); segmented varlen launches map it
// to the global position-major unit seg * KU + u (the caller has checked that
// this is below n_units)
__device__ __forceinline__ UnitRef unit_ref(const Geom& G, int u) {
  UnitRef R;
  if (G.pos_off != nullptr) {
    // position p of the unit: the largest p in [P0, P1] with pos_off[p] <= ug
    // (P0, P1 the positions of this segment's and the next one's first unit)
    const int ug = G.seg * G.KU + u;
    int lo = G.seg_pos[2 * G.seg], hi = G.seg_pos[2 * G.seg + 2];
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (G.pos_off[mid] <= ug) lo = mid; else hi = mid - 1;
    }
    R.seq = G.order[ug - G.pos_off[lo]];
    R.n = lo;
    const int s0 = G.cu_clamped[R.seq], s1 = G.cu_clamped[R.seq + 1];
    R.row0 = static_cast<int64_t>(s0) + static_cast<int64_t>(R.n) * kC;
    R.len = min(kC, static_cast<int>(s1 - R.row0));
    return R;
  }
  if (G.cu == nullptr) {
    // dense: units are (sequence, chunk) of the segment [n0, n0 + NTS)
    R.seq = u / G.NTS;
    R.n = G.n0 + (u - R.seq * G.NTS);
    R.row0 = static_cast<int64_t>(R.seq) * G.T + static_cast<int64_t>(R.n) * kC;
    R.len = min(kC, G.T - R.n * kC);
  } else {
    // largest s with chunk_off[s] <= u (chunk_off is non-decreasing)
    int lo = 0, hi = G.N - 1;
    while (lo < hi) {
      int mid = (lo + hi + 1) >> 1;
      if (G.chunk_off[mid] <= u) lo = mid; else hi = mid - 1;
    }
    R.seq = lo;
    R.n = u - G.chunk_off[lo];
    int s0 = G.cu_clamped[lo], s1 = G.cu_clamped[lo + 1];
    R.row0 = static_cast<int64_t>(s0) + static_cast<int64_t>(R.n) * kC;
    R.len = min(kC, static_cast<int>(s1 - R.row0));
  }
  return R;
}

// The chunks of one chain that a state launch walks.  chain_unit(G, c, n) is
// the workspace slot of its n-th chunk in the launch; rows tok0 + 64 n on,
// seq_len - 64 n of them valid.  The walk starts from h0 (from_h0) or from
// the state the previous segment left in ht; an inactive chain (a segmented
// varlen launch holding none of its chunks) touches nothing.
struct ChainRef {
  int seq, u0, nchunks, seq_len;
  int64_t tok0;
  int rank, p0;   // segmented varlen: longest-first rank, first chunk position
  bool from_h0, active;
};

// rank: the chain's sequence slot of the state grid (varlen: its rank in the
// longest-first order; dense: the batch row)
__device__ __forceinline__ ChainRef chain_ref(const Geom& G, int rank) {
  ChainRef c;
  c.seq = (G.order != nullptr) ? G.order[rank] : rank;
  c.rank = rank;
  c.p0 = 0;
  c.from_h0 = true;
  c.active = true;
  if (G.cu == nullptr) {
    c.u0 = c.seq * G.NTS;
    c.nchunks = G.NTS;
    c.tok0 = static_cast<int64_t>(c.seq) * G.T + static_cast<int64_t>(G.n0) * kC;
    c.seq_len = G.T - G.n0 * kC;
  } else if (G.pos_off == nullptr) {
    c.u0 = G.chunk_off[c.seq];
    c.nchunks = G.chunk_off[c.seq + 1] - c.u0;
    c.tok0 = G.cu_clamped[c.seq];
    c.seq_len = G.cu_clamped[c.seq + 1] - G.cu_clamped[c.seq];
  } else {
    // The chain's units pos_off[p] + rank increase with p; this segment holds
    // positions [p_lo, p_hi) of them: from the first segment unit's (P0, R0)
    // and the next segment's (P1, R1), p_lo = P0 + (rank < R0), p_hi = P1 +
    // (rank < R1), clamped to the chain's chunk count.
    const int ni = G.chunk_off[c.seq + 1] - G.chunk_off[c.seq];
    const int P0 = G.seg_pos[2 * G.seg], R0 = G.seg_pos[2 * G.seg + 1];
    const int P1 = G.seg_pos[2 * G.seg + 2], R1 = G.seg_pos[2 * G.seg + 3];
    const int p_lo = P0 + (rank < R0 ? 1 : 0);
    const int p_hi = min(P1 + (rank < R1 ? 1 : 0), ni);
    c.p0 = p_lo;
    c.u0 = 0;
    c.nchunks = max(p_hi - p_lo, 0);
    const int s0 = G.cu_clamped[c.seq];
    c.tok0 = static_cast<int64_t>(s0) + static_cast<int64_t>(p_lo) * kC;
    c.seq_len = G.cu_clamped[c.seq + 1] - s0 - p_lo * kC;
    c.from_h0 = (p_lo == 0);
    // an empty sequence's final state (h0) is written by the first segment
    c.active = c.nchunks > 0 || (ni == 0 && G.seg == 0);
  }
  return c;
}

__device__ __forceinline__ int chain_unit(const Geom& G, const ChainRef& c, int n) {
  if (G.pos_off != nullptr) return G.pos_off[c.p0 + n] + c.rank - G.seg * G.KU;
  return c.u0 + n;
}

// ----------------------------------------------------------------------------
// Intra-chunk work of one chunk-head (device function, per wave W)
// ----------------------------------------------------------------------------
template <int DK, int DV, bool EXACT>
struct IntraSmem {
  typedef typename Prec<EXACT>::st st;
  static constexpr int PK = DK + 8;   // row pitch (elements) of [C][DK] buffers
  static constexpr int PC = kC + 8;   // row pitch of [*][C] buffers
  static constexpr int R1 = (kC * PK > DK * PC) ? kC * PK : DK * PC;
  // region 1, two lives: k*Cf (scores) -> (beta*gamma*k)^T (W product)
  st r1[R1];
  st BVt[DV * PC];        // (beta*v)^T, rows = channel
  // T = (I+L)^-1 (wave w writes row block w after barrier #2).  Before that
  // barrier the same bytes hold each wave's per-tile factors and, once its
  // score tiles are done, its diagonal L block (both wave-local).
  st Tm[kC * PC];
  st Lmb[6][16][16];      // off-diagonal L blocks, row-major; block (R,j) at R(R-1)/2+j
  st Tdg[4][16][16];      // diagonal T blocks, row-major
  float tot[4][DK];       // per-tile log2 decay totals, slot order
  // Factor rows of wave w (2^pre, 2^post, 2^-D, then M(w,w-2) from w = 2 on
  // and M(w,w-3) from w = 3 on): rows FR0[w] .. FR0[w+1]-1 of DK floats.
  static constexpr int FR0[5] = {0, 3, 6, 10, 15};
  __device__ float* fac(int w, int k) { return reinterpret_cast<float*>(Tm) + (FR0[w] + k) * DK; }
  // the diagonal L block of wave w, fp32 [16][20]: over the wave's own factor
  // rows when they are large enough, else after all factor rows
  static constexpr bool LD_IN_FAC = 3 * DK >= 16 * 20;
  __device__ float (*Ld(int w))[20] {
    float* base = LD_IN_FAC ? fac(w, 0) : reinterpret_cast<float*>(Tm) + FR0[4] * DK + w * 16 * 20;
    return reinterpret_cast<float (*)[20]>(base);
  }
  static_assert(sizeof(st) * kC * PC >= sizeof(float) * (FR0[4] * DK + (LD_IN_FAC ? 0 : 4 * 16 * 20)),
                "factor rows and diagonal L blocks exceed the T buffer");
};

// The intra kernel stages fp32 gate rows through LDS when q, k, v are 16-bit
// and g is fp32 (BF16_F32GATES, the cc_scan seam), outside the fused
// prologue and the exact mode.
template <int DTQ, int DTG, bool EXACT, bool PRO>
struct IntraG32 {
  static constexpr bool value = DTG == 0 && DTQ != 0 && !EXACT && !PRO;
};

// Shared memory of the intra kernel: IntraSmem, or the larger staging area
// the fused prologue needs (64 rows of g plus 4 waves x 3 tensors x (16 +
// history) rows) or the fp32-gate staging (64 fp32 g rows, 64 rows of q and
// of k), whichever is bigger.
template <int DK, int DV, bool EXACT, bool PRO, bool G32>
struct IntraLds;

// channel of slot index s
__device__ __forceinline__ int slot_index_channel(int s) {
  return slot_channel(s >> 5, (s >> 3) & 3, s & 7);
}

// Where a wave of the fused-prologue kernel parks its lane's convolved q and
// k words of K step j (8 bf16 each, the slot order of the score operands)
// when its tile takes the anchored path: this chunk-head's U and W slots of
// its own row tile, which the final products write only after barrier #3
// (every read of the parked words precedes barrier #2).
template <int DK>
__device__ __forceinline__ int64_t park_k_slot(int64_t chead, int W, int j, int l) {
  return (chead * (kC / 16) * (DK / 32) + (W * (DK / 32) + j)) * 512 + l * 8;
}
template <int DK>
__device__ __forceinline__ int64_t park_q_slot(int64_t chead, int W, int j, int l) {
  return (chead * (kC / 16) * (DK / 16) + (W * (DK / 16) + 2 * j)) * 256 + l * 8;
}

// One K step (channels 32j .. 32j+31) of the diagonal tile of row tile W when
// the tile's decay passes 2^-100 in some channel and no single row factor pair
// fits fp32.  The pair (c, i), c > i, splits at the highest bit h where c and
// i differ, through the anchor row a = (i | (2^h - 1)) in [i, c):
// 2^(G_c - G_a) * 2^(G_a - G_i), both factors <= 1 whatever the decay.  At
// level h the key rows with bit h clear carry 2^(G_a - G_i), the query rows
// with bit h set 2^(G_c - G_a), every other row 0, and the level's products
// are kept for its own pairs only; the diagonal (Aqk) has factor 1 (pass
// hb = -1).  Each pass reloads k, q and g and recomputes the tile-local
// cumsum (the same scan, so the same values).  With the fused prologue q and
// k come from the slots the wave parked them in (pq_slot, pk_slot below), g
// from memory as always.  acc holds the lane's Akk and Aqk accumulators of
// the tile (4 + 4) and is returned updated.  Not unrolled, and run after the
// score loop (whose row slices and factors are then dead): the rare path's
// temporaries do not add to the registers of the common path.
template <int DK, int DTQ, int DTG, bool EXACT, int W, bool PRO>
__device__ __forceinline__ f8 extreme_diag_step(const IntraArgs* ap, const int j, const int64_t chead,
                                               const int len, const int64_t row0, const int h, f8 acc) {
  typedef typename Prec<EXACT>::st st;
  constexpr int NJ = DK / 32;
  const IntraArgs& a = *ap;
  const int l = threadIdx.x & 63, r = l & 15, gq = l >> 4;
  const int c = 16 * W + r;
  const bool valid = c < len;
  const int64_t bq = ((row0 + c) * a.geom.H + h) * DK;
  auto decay2 = [&](float z) -> float {
    if constexpr (DTG == 0) {
      if (a.gates_alpha) {
        const bool dn = z < 1.17549435e-38f;
        return __builtin_amdgcn_logf(dn ? z * 4294967296.0f : z) - (dn ? 32.0f : 0.0f);
      }
    }
    return z * kLog2e;
  };
#pragma unroll 1
  for (int hb = -1; hb < 4; ++hb) {
    const int an = (hb < 0) ? r : (r & ~((2 << hb) - 1)) | ((1 << hb) - 1);   // anchor of this row
    const bool key = (hb < 0) || ((r >> hb) & 1) == 0;
    uint4 pq = {0, 0, 0, 0}, pk = {0, 0, 0, 0};
    if constexpr (PRO) {
      pq = *reinterpret_cast<const uint4*>(static_cast<const st*>(a.U) + park_q_slot<DK>(chead, W, j, l));
      pk = *reinterpret_cast<const uint4*>(static_cast<const st*>(a.W) + park_k_slot<DK>(chead, W, j, l));
    }
    f8 A, Bk, Bq;
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int ch0 = 32 * j + 4 * gq + 16 * hf;
      f4 x = {0, 0, 0, 0}, y = {0, 0, 0, 0}, z = {0, 0, 0, 0};
      if (valid) {
        if constexpr (PRO) {
          x = unpack4<DTQ>(hf ? uint2{pq.z, pq.w} : uint2{pq.x, pq.y});
          y = unpack4<DTQ>(hf ? uint2{pk.z, pk.w} : uint2{pk.x, pk.y});
        } else {
          x = ld4<DTQ>(a.q, bq + ch0);
          y = ld4<DTQ>(a.k, bq + ch0);
        }
        z = ld4<DTG>(a.g, bq + ch0);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int ee = 4 * hf + e;
        const float gt = row_scan16(valid ? decay2(z[e]) : 0.f);
        const float ga = __shfl(gt, (l & 48) | an, 64);
        const float f = (hb < 0) ? 1.f : fast_exp2(key ? ga - gt : gt - ga);
        A[ee] = key ? y[e] * f : 0.f;
        Bk[ee] = (hb < 0 || key) ? 0.f : y[e] * f;
        Bq[ee] = (hb < 0) ? x[e] * a.scale : key ? 0.f : x[e] * a.scale * f;
      }
    }
    f4 tK = {0, 0, 0, 0}, tQ = {0, 0, 0, 0};
    if constexpr (EXACT) {
      tK = mma32(tK, A, Bk);
      tQ = mma32(tQ, A, Bq);
    } else {
      b8 ah, al, kh, kl;
      split_bf16(A, ah, al);
      split_bf16(Bk, kh, kl);
      tK = mma32_bf16(tK, ah, kh);
      tK = mma32_bf16(tK, ah, kl);
      tK = mma32_bf16(tK, al, kh);
      split_bf16(Bq, kh, kl);
      tQ = mma32_bf16(tQ, ah, kh);
      tQ = mma32_bf16(tQ, ah, kl);
      tQ = mma32_bf16(tQ, al, kh);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int ii = 4 * gq + i;
      if (hb < 0) {
        if (r == ii) acc[4 + i] += tQ[i];
      } else if (r > ii && ((r ^ ii) >> hb) == 1) {
        acc[i] += tK[i];
        acc[4 + i] += tQ[i];
      }
    }
  }
  return acc;
}

template <int DK, int DV, int DTQ, int DTG, bool EXACT, int W, bool PRO>
__device__ __forceinline__ void intra_chunk(const IntraArgs& a, const UnitRef& U, const int h,
                                            const int64_t chead, IntraSmem<DK, DV, EXACT>& sm) {
  typedef typename Prec<EXACT>::st st;
  typedef typename Prec<EXACT>::v8 v8;
  typedef typename Prec<EXACT>::v4 v4;
  typedef IntraSmem<DK, DV, EXACT> SM;
  constexpr int NJ = DK / 32;     // 32-wide K steps over dk
  constexpr int NJV = DV / 32;
  constexpr int PK = SM::PK;
  constexpr int PC = SM::PC;
  const int tid = threadIdx.x;
  const int l = tid & 63, r = l & 15, gq = l >> 4;
  const int H = a.geom.H;
  st* const oW = static_cast<st*>(a.W);
  st* const oU = static_cast<st*>(a.U);
  st* const oAQ = static_cast<st*>(a.AQ);
  st* const oGQ = static_cast<st*>(a.GQ);
  st* const oLK = static_cast<st*>(a.LK);

  const int c = 16 * W + r;           // my row inside the chunk
  const bool valid = c < U.len;
  const int64_t tok = U.row0 + c;
  const int64_t bq = (tok * H + h) * DK;

  // ---- loads (slot order), masked rows are zero -----------------------------
  // 16-bit q, k, v (and g) rows are first copied into LDS by direct
  // global->LDS loads: each instruction moves whole rows (1 KiB, fully
  // coalesced), where per-lane loads of the slot order would touch 16 rows x
  // 32 B per instruction.  Each wave copies only its own 16 rows, so a
  // wave-local wait suffices; 16-byte chunks are XOR-swizzled by row so the
  // slot-order reads below are spread over the LDS banks.  The staging area
  // aliases the buffers of the later phases (barrier before their first use).
  // fp32 g rows are staged the same way when q, k, v are 16-bit; the exact
  // mode's fp32 tensors are loaded per lane.
  constexpr bool STQ = (DTQ != 0);
  // fp32 gates with 16-bit q, k, v (G32): g is staged too, in fp32 rows of
  // twice the bytes, each copy instruction moving RPI / 2 of them
  constexpr bool G32 = IntraG32<DTQ, DTG, EXACT, PRO>::value;
  constexpr bool STG = (DTG != 0) || G32;
  constexpr int ROWB = DK * 2;          // bytes per staged 16-bit row
  constexpr int NCH = ROWB / 16;        // 16-byte chunks per row
  constexpr int RPI = 1024 / ROWB;      // rows per copy instruction
  constexpr int ROWG = G32 ? 2 * ROWB : ROWB;   // bytes per staged g row
  constexpr int NCHG = ROWG / 16;
  constexpr int RPIG = 1024 / ROWG;
  // Without the fused prologue three [64][DK] tensors are staged at a time:
  // q, k and g, then v in g's rows once the wave has read its g.
  static_assert(PRO || !(STQ || STG) || IntraLds<DK, DV, EXACT, PRO, G32>::kBytes >= kC * (2 * ROWB + ROWG),
                "staging area exceeds the shared buffers");
  static_assert(DK == DV, "staging assumes dk == dv");
  static_assert(!PRO || (DTQ == 1 && !EXACT), "the fused prologue stages bf16 projections");
  unsigned char* const stg = reinterpret_cast<unsigned char*>(&sm);
  // With the fused prologue (PRO) each wave stages, for q, k and v, RPI rows
  // before its own 16 (the convolution's history) into rows of its own: HR
  // rows per wave and tensor after the 64 rows of g.
  constexpr int HR = 16 + RPI;
  auto stg_row = [&](int t, int row) -> unsigned char* {
    if constexpr (PRO) {
      if (t == 2) return stg + row * ROWB;
      const int tt = (t == 3) ? 2 : t;   // q, k, v
      return stg + (kC + (tt * 4 + W) * HR + (row - 16 * W + RPI)) * ROWB;
    } else if constexpr (G32) {
      // g rows first; a wave's 16 v rows, dense, over its own g rows
      if (t == 2) return stg + row * ROWG;
      if (t == 3) return stg + (row & ~15) * ROWG + (row & 15) * ROWB;
      return stg + kC * ROWG + (t * kC + row) * ROWB;
    } else {
      return stg + ((t == 3 ? 2 : t) * kC + row) * ROWB;   // v over g
    }
  };
  // beta first: its latency hides behind the row copies.  Copy order g, k, q,
  // v: with all four staged (SPLIT) the waits below are partial (vmcnt retires
  // in issue order), so the decay scan runs while k, q and v are still
  // arriving and the k/q decay factors while v is.
  constexpr bool SPLIT = STQ && STG;
  constexpr int NPER = 16 / RPI;        // copies per tensor per wave
  constexpr int NQKV = PRO ? NPER + 1 : NPER;   // copies per q, k, v (PRO: one of history rows)
  // (unconditional load of a valid row, masked after the waits: a load
  // inside a branch is waited for at the branch's end)
  float beta_c;
  if constexpr (DTG == 0) {
    const int64_t bi = (U.row0 + min(c, U.len - 1)) * H + h;
    if (a.gates_alpha) {
      // cc_scan's beta32 row: the mean of its 32 columns, summed in column
      // order.  Lane group gq loads columns 8 gq .. 8 gq + 7 (two 16-byte
      // loads), and the running sum passes from group to group: at step s
      // group s adds its eight columns to the sum of the groups before it.
      const f4* b32 = reinterpret_cast<const f4*>(static_cast<const float*>(a.beta) + bi * 32 + 8 * gq);
      const f4 bl = b32[0], bh = b32[1];
      float sb = 0.f, t = 0.f;
#pragma unroll
      for (int st = 0; st < 4; ++st) {
        t = sb;
#pragma unroll
        for (int e = 0; e < 4; ++e) t += bl[e];
#pragma unroll
        for (int e = 0; e < 4; ++e) t += bh[e];
        sb = __shfl(t, r + 16 * st, 64);
      }
      beta_c = sb * (1.0f / 32.0f);
    } else {
      beta_c = ld1<DTG>(a.beta, bi);
    }
  } else {
    beta_c = ld1<DTG>(a.beta, (U.row0 + min(c, U.len - 1)) * H + h);
  }
  // PRO: conv taps of this lane's channels PL*l .. PL*l + PL-1 and, for the
  // first chunk of a sequence (wave 0), the carried inputs before it; loaded
  // before the row copies, so the copies' partial waits cover them
  constexpr int PL = DK / 64;
  constexpr int KM = kFusedConvTaps;
  float cwv[3][KM][PL];
  float hist[3][KM - 1][PL];
  if constexpr (PRO) {
    const int64_t HD = static_cast<int64_t>(H) * DK;
#pragma unroll
    for (int tt = 0; tt < 3; ++tt)
#pragma unroll
      for (int i = 0; i < KM; ++i) {
        const float* wp = a.cw[tt] + min(i, a.K - 1) * HD + h * DK + PL * l;
        if constexpr (PL == 2) {
          const float2 w2 = *reinterpret_cast<const float2*>(wp);
          cwv[tt][i][0] = w2.x;
          cwv[tt][i][1] = w2.y;
        } else {
          cwv[tt][i][0] = *wp;
        }
      }
    if constexpr (W == 0) {
#pragma unroll
      for (int tt = 0; tt < 3; ++tt)
#pragma unroll
        for (int j = 0; j < KM - 1; ++j)
#pragma unroll
          for (int p = 0; p < PL; ++p) hist[tt][j][p] = 0.f;
      if (U.n == 0) {
        // row j - (KM-1) of the chunk is buffer row K-1 + j - (KM-1) (oldest first)
#pragma unroll
        for (int tt = 0; tt < 3; ++tt) {
          if (a.cb[tt] == nullptr) continue;
#pragma unroll
          for (int j = 0; j < KM - 1; ++j) {
            const int br = a.K - 1 + j - (KM - 1);
            if (br < 0) continue;
            const float* bp = a.cb[tt] + (static_cast<int64_t>(U.seq) * (a.K - 1) + br) * HD + h * DK + PL * l;
#pragma unroll
            for (int p = 0; p < PL; ++p) hist[tt][j][p] = bp[p];
          }
        }
      }
    }
  }
  // direct global->LDS copies of this wave's rows of tensor t (non-temporal:
  // each row is read by this chunk-head only, and kept in L2 it would
  // displace workspace lines; config 1 225 -> 215 us when introduced)
  auto stage_rows = [&](const int t) {
    const unsigned char* src = static_cast<const unsigned char*>(t == 0 ? a.q : t == 1 ? a.k : t == 2 ? a.g : a.v);
    const bool g32 = G32 && t == 2;
    const int rowb = g32 ? ROWG : ROWB, nch = g32 ? NCHG : NCH, rpi = g32 ? RPIG : RPI;
    const int nc = (t == 2) ? 16 / rpi : NQKV;
    const int r0 = (PRO && t != 2) ? 16 * W - RPI : 16 * W;         // first row copied
#pragma unroll
    for (int i = 0; i < nc; ++i) {
      const int row = r0 + rpi * i + l / nch;                       // chunk row this lane copies
      const int cidx = (l % nch) ^ (row & (nch - 1));               // source chunk of LDS chunk l % nch
      // rows past the end re-read a valid row; history rows before a
      // sequence's first chunk (replaced by the carried inputs) read row 0
      int rv = min(row, U.len - 1);
      if (PRO && U.n == 0) rv = max(rv, 0);
      const int64_t srow = U.row0 + rv;
      const unsigned char* gsrc = src + (srow * H + h) * static_cast<int64_t>(rowb) + cidx * 16;
      unsigned char* ldst = stg_row(t, r0 + rpi * i);
      __builtin_amdgcn_global_load_lds(gsrc, ldst, 16, 0, kCpolStream);
    }
  };
  // v goes into g's rows once the wave has read its g (below) when g is staged
  constexpr bool V_LATE = !PRO && STG;
  if constexpr (STQ || STG) {
#pragma unroll
    for (int oi = 0; oi < 4; ++oi) {
      const int t = (oi == 0) ? 2 : (oi == 1) ? 1 : (oi == 2) ? 0 : 3;  // 0 q, 1 k, 2 g, 3 v
      if ((t == 2) ? !STG : !STQ) continue;
      if (V_LATE && t == 3) continue;
      stage_rows(t);
    }
    if constexpr (!SPLIT) {
      wait_vmem_all();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    }
  }
  // four channels ch0 = 32j + 16hf + 4gq .. +3 of this lane's row from
  // staging, all 2 NJ of them for tensor t (read untracked, then settled)
  auto stg_read_all = [&](int t, uint2 (&w)[2 * NJ]) {
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int ci = 4 * j + 2 * hf + (gq >> 1);
        const int pc = ci ^ (c & (NCH - 1));
        w[2 * j + hf] = ds_read_b64_raw(stg_row(t, c) + pc * 16 + (gq & 1) * 8);
      }
    lds_settle(w);
  };
  // Rows past the chunk's end (staged copies of a real row) need no masking
  // except g and beta: beta = 0 zeroes their rows of L, W and U and hence of
  // v~, and their o rows are never stored; g = 0 keeps them out of the
  // chunk's decay.
  float kr[NJ][8], qr[NJ][8], kc[NJ][8], Gt[NJ][8];
  float vr[NJV][8];
  // a gate value in log2 units: g log2(e), or with alpha gates (cc_scan:
  // g holds alpha) log2(alpha) directly by the hardware base-2 logarithm.
  // That instruction flushes a denormal input to zero (log2 = -inf, and
  // -inf - -inf = NaN in the decay factors): a denormal alpha is scaled by
  // 2^32 first and 32 taken off the logarithm.
  auto decay2 = [&](float z) -> float {
    if constexpr (DTG == 0) {
      if (a.gates_alpha) {
        const bool dn = z < 1.17549435e-38f;
        return __builtin_amdgcn_logf(dn ? z * 4294967296.0f : z) - (dn ? 32.0f : 0.0f);
      }
    }
    return z * kLog2e;
  };

  // g -> log2 decay, then the tile-local inclusive scan
  if constexpr (SPLIT) {
    wait_vmem<(V_LATE ? 2 : 3) * NQKV>();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
  }
  uint2 sw[2 * NJ];
  u32x4 sg[G32 ? 2 * NJ : 1];
  if constexpr (G32) {
    // four fp32 channels ch0 = 32j + 16hf + 4gq .. +3: one 16-byte chunk
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int ci = 8 * j + 4 * hf + gq;
        sg[2 * j + hf] = ds_read_b128_raw(stg_row(2, c) + (ci ^ (c & (NCHG - 1))) * 16);
      }
    lds_settle(sg);
  } else if constexpr (STG) {
    stg_read_all(2, sw);
  }
  // g is in registers (settled): v's copies may now overwrite its rows; they
  // are the newest copies, so the waits below for k, q and then v are as
  // before
  if constexpr (V_LATE) stage_rows(3);
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      f4 z = {0, 0, 0, 0};
      if constexpr (G32) z = __builtin_bit_cast(f4, sg[2 * j + hf]);
      else if constexpr (STG) z = unpack4<DTG>(sw[2 * j + hf]);
      else if (valid) z = ld4<DTG>(a.g, bq + 32 * j + 4 * gq + 16 * hf);
#pragma unroll
      for (int e = 0; e < 4; ++e) Gt[j][4 * hf + e] = valid ? decay2(z[e]) : 0.f;
    }
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) Gt[j][e] = row_scan16(Gt[j][e]);
  // PRO: whether this wave's tile takes the anchored path (the same test as
  // `extreme` below), known before the convolution so that the wave can park
  // its convolved q and k for that path as soon as it reads them
  bool ext_pro = false;
  if constexpr (PRO) {
    float dm = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) dm = fminf(dm, row_bcast<15>(Gt[j][e]));
    ext_pro = __any(dm < -100.f);
  }

  // k, q and the two decay factors.  Each group's results are tied to an
  // empty asm statement before the next group's wait: otherwise the compiler
  // sinks the arithmetic to its first use, past the staging barrier, and the
  // copies still in flight hide nothing.
  if constexpr (SPLIT) {
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) asm volatile("" : "+v"(Gt[j][e]));
    if constexpr (!PRO) {
      wait_vmem<NPER>();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    }
  }
  if constexpr (PRO) {
    // Fused prologue, k first (its rows arrive first), then q, then v: per
    // row out = sum_i w[i] x[row - i] (fp32, taps in order), swish, for q
    // and k times 1 / (||row|| + 1e-12), rounded to bf16 and written over
    // the staged row -- the arithmetic of kda_prologue_kernel, lane for lane.
    auto conv = [&](const int t, const int tt, const bool nrm) {
      constexpr int NR = 15 + KM;     // rows 16W - (KM-1) .. 16W + 15
      const int ci = (PL * l) >> 3, cb = ((PL * l) & 7) * 2;
      unsigned raw[NR];
#pragma unroll
      for (int j = 0; j < NR; ++j) {
        const int row = 16 * W - (KM - 1) + j;
        const unsigned char* p = stg_row(t, row) + (ci ^ (row & (NCH - 1))) * 16 + cb;
        raw[j] = (PL == 2) ? ds_read_b32_raw(p) : ds_read_u16_raw(p);
      }
      lds_settle(raw);
      float xs[NR][PL];
#pragma unroll
      for (int j = 0; j < NR; ++j) {
        xs[j][0] = bf16_to_f32(static_cast<u16>(raw[j] & 0xFFFFu));
        if constexpr (PL == 2) xs[j][1] = bf16_to_f32(static_cast<u16>(raw[j] >> 16));
      }
      if constexpr (W == 0) {
        if (U.n == 0) {
#pragma unroll
          for (int j = 0; j < KM - 1; ++j)
#pragma unroll
            for (int p = 0; p < PL; ++p) xs[j][p] = hist[tt][j][p];
        }
      }
      float sv[16][PL], ss[16];
#pragma unroll
      for (int r2 = 0; r2 < 16; ++r2) {
        ss[r2] = 0.f;
#pragma unroll
        for (int p = 0; p < PL; ++p) {
          float acc = 0.f;
#pragma unroll
          for (int i = 0; i < KM; ++i)
            if (i < a.K) acc = fmaf(cwv[tt][i][p], xs[r2 + KM - 1 - i][p], acc);
          sv[r2][p] = acc * sigmoid_f32(acc);
          ss[r2] = fmaf(sv[r2][p], sv[r2][p], ss[r2]);
        }
      }
      if (nrm) {
        float tot[16];
        wave_rowsums16(ss, tot);
#pragma unroll
        for (int r2 = 0; r2 < 16; ++r2) {
          const float sc = inv_l2_f32(tot[r2]);
#pragma unroll
          for (int p = 0; p < PL; ++p) sv[r2][p] *= sc;
        }
      }
#pragma unroll
      for (int r2 = 0; r2 < 16; ++r2) {
        const int row = 16 * W + r2;
        unsigned char* p = stg_row(t, row) + (ci ^ (row & (NCH - 1))) * 16 + cb;
        if constexpr (PL == 2) ds_write_b32_raw(p, pack_bf16x2(sv[r2][0], sv[r2][1]));
        else ds_write_b16_raw(p, cvt_bf16(sv[r2][0]));
      }
    };
    if constexpr (SPLIT) {
      wait_vmem<2 * NQKV>();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    }
    conv(1, 1, true);
    if constexpr (SPLIT) {
      wait_vmem<NQKV>();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    }
    conv(0, 0, true);
    if constexpr (SPLIT) {
      wait_vmem<0>();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    }
    conv(3, 2, false);
  }
  uint2 sq[2 * NJ];
  if constexpr (STQ) {
    stg_read_all(0, sq);
    stg_read_all(1, sw);
  }
  if constexpr (PRO) {
    // The anchored path of an extreme tile (below) re-reads q and k per
    // level; with the fused prologue they exist only here (the convolved bf16
    // rows in LDS are overwritten after the staging barrier).  A wave whose
    // tile takes that path parks its lane's q and k words in slots of the
    // workspace that are written only later (park_q_slot, park_k_slot).
    if (ext_pro) {
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        *reinterpret_cast<uint4*>(oU + park_q_slot<DK>(chead, W, j, l)) =
            uint4{sq[2 * j].x, sq[2 * j].y, sq[2 * j + 1].x, sq[2 * j + 1].y};
        *reinterpret_cast<uint4*>(oW + park_k_slot<DK>(chead, W, j, l)) =
            uint4{sw[2 * j].x, sw[2 * j].y, sw[2 * j + 1].x, sw[2 * j + 1].y};
      }
    }
  }
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int ch0 = 32 * j + 4 * gq + 16 * hf;
      f4 x = {0, 0, 0, 0}, y = {0, 0, 0, 0};
      if constexpr (STQ) {
        x = unpack4<DTQ>(sq[2 * j + hf]);
        y = unpack4<DTQ>(sw[2 * j + hf]);
      } else if (valid) {
        x = ld4<DTQ>(a.q, bq + ch0);
        y = ld4<DTQ>(a.k, bq + ch0);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        qr[j][4 * hf + e] = x[e];
        kr[j][4 * hf + e] = y[e];
      }
    }
  if (a.scale != 1.f) {
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) qr[j][e] *= a.scale;
  }
  float dmin = 0.f;
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float gt = Gt[j][e];
      const float dw = row_bcast<15>(gt);
      dmin = fminf(dmin, dw);
      const float R = fast_exp2(gt);
      kc[j][e] = kr[j][e] * fast_exp2(dw - gt);
      kr[j][e] *= R;
      qr[j][e] *= R;
    }

  // v
  if constexpr (SPLIT) {
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) asm volatile("" : "+v"(kc[j][e]), "+v"(kr[j][e]), "+v"(qr[j][e]));
    wait_vmem<0>();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
  }
  if constexpr (STQ) stg_read_all(3, sw);
#pragma unroll
  for (int j = 0; j < NJV; ++j)
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      f4 w = {0, 0, 0, 0};
      if constexpr (STQ) w = unpack4<DTQ>(sw[2 * j + hf]);
      else if (valid) w = ld4<DTQ>(a.v, (tok * H + h) * DV + 32 * j + 4 * gq + 16 * hf);
#pragma unroll
      for (int e = 0; e < 4; ++e) vr[j][4 * hf + e] = w[e];
    }
  if (!valid) beta_c = 0.f;
  // every wave has read its staged rows before any buffer they alias is written
  if constexpr (STQ || STG) lds_barrier();

  // beta * v  -> BVt (channel-major); tile totals; k*Cf -> region 1
#pragma unroll
  for (int j = 0; j < NJV; ++j)
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int ch0 = 32 * j + 4 * gq + 16 * hf;
#pragma unroll
      for (int e = 0; e < 4; ++e) sm.BVt[(ch0 + e) * PC + c] = st(beta_c * vr[j][4 * hf + e]);
    }
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    f8 x, tj;
#pragma unroll
    for (int e = 0; e < 8; ++e) { x[e] = kc[j][e]; tj[e] = Gt[j][e]; }
    if (r == 15) *reinterpret_cast<f8*>(&sm.tot[W][32 * j + 8 * gq]) = tj;
    *reinterpret_cast<v8*>(&sm.r1[c * PK + 32 * j + 8 * gq]) = cvt8<EXACT>(x);
  }
  // a tile whose decay total passes 2^-100 in some channel: anchored path
  const bool extreme = __any(dmin < -100.f);
  // The diagonal tile's operands are k*Cf and (k or q)*R*2^-D.  When every
  // channel's tile total D is above -12 and |k*Cf|, |k*R|, |q*R| <= 8 they
  // fit fp16 (< 2^15) and the tile runs on one fp16 MFMA pair like the
  // off-diagonal ones; otherwise on bf16 hi/lo.
  bool diag16 = false;
  if constexpr (!EXACT) {
    float mx = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fmaxf(fabsf(kc[j][e]), fmaxf(fabsf(kr[j][e]), fabsf(qr[j][e]))));
    diag16 = !__any(dmin < -12.f || !(mx <= 8.f));
  }
  lds_barrier();  // #1: tot, k*Cf, BVt

  // ---- per-channel constants of this tile (wave-local) -----------------------
#pragma unroll
  for (int s0 = l; s0 < DK; s0 += 64) {
    const float tt[4] = {sm.tot[0][s0], sm.tot[1][s0], sm.tot[2][s0], sm.tot[3][s0]};
    float pre = 0.f, post = 0.f;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      if (t < W) pre += tt[t];
      if (t > W) post += tt[t];
    }
    sm.fac(W, 0)[s0] = fast_exp2(pre);
    sm.fac(W, 1)[s0] = fast_exp2(post);
    sm.fac(W, 2)[s0] = fast_exp2(-tt[W]);
    if constexpr (W >= 2) sm.fac(W, 3)[s0] = fast_exp2(tt[W - 1]);
    if constexpr (W >= 3) sm.fac(W, 4)[s0] = fast_exp2(tt[W - 1] + tt[W - 2]);
    if constexpr (W == 0) a.GC[chead * DK + slot_index_channel(s0)] = fast_exp2(tt[0] + tt[1] + tt[2] + tt[3]);
  }
  __builtin_amdgcn_wave_barrier();  // this wave reads back its own fac[W] below

  // ---- scores: Akk^T / Aqk^T tiles (s, W), s <= W ----------------------------
  f4 accK[W + 1], accQ[W + 1];
#pragma unroll
  for (int s = 0; s <= W; ++s) { accK[s] = f4{0, 0, 0, 0}; accQ[s] = f4{0, 0, 0, 0}; }
  v8 lk[NJ];  // lambda*k, packed operand precision
  v8 bw[NJ];  // beta*gamma*k, packed operand precision

#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int sb = 32 * j + 8 * gq;
    const f8 P = *reinterpret_cast<const f8*>(&sm.fac(W, 0)[sb]);
    const f8 Q = *reinterpret_cast<const f8*>(&sm.fac(W, 1)[sb]);
    const f8 iD = *reinterpret_cast<const f8*>(&sm.fac(W, 2)[sb]);
    f8 krj, qrj;
#pragma unroll
    for (int e = 0; e < 8; ++e) { krj[e] = kr[j][e]; qrj[e] = qr[j][e]; }

    // off-diagonal tiles: A = k*Cf of key tile s (LDS), B = row operand of tile W
    if constexpr (W >= 1) {
      constexpr int s = W - 1;
      const v8 A = *reinterpret_cast<const v8*>(&sm.r1[(16 * s + r) * PK + sb]);
      accK[s] = mma32(accK[s], A, cvt8<EXACT>(krj));
      accQ[s] = mma32(accQ[s], A, cvt8<EXACT>(qrj));
    }
    if constexpr (W >= 2) {
      constexpr int s = W - 2;
      const f8 M2 = *reinterpret_cast<const f8*>(&sm.fac(W, 3)[sb]);
      const v8 A = *reinterpret_cast<const v8*>(&sm.r1[(16 * s + r) * PK + sb]);
      accK[s] = mma32(accK[s], A, cvt8<EXACT>(krj * M2));
      accQ[s] = mma32(accQ[s], A, cvt8<EXACT>(qrj * M2));
    }
    if constexpr (W >= 3) {
      constexpr int s = W - 3;
      const f8 M3 = *reinterpret_cast<const f8*>(&sm.fac(W, 4)[sb]);
      const v8 A = *reinterpret_cast<const v8*>(&sm.r1[(16 * s + r) * PK + sb]);
      accK[s] = mma32(accK[s], A, cvt8<EXACT>(krj * M3));
      accQ[s] = mma32(accQ[s], A, cvt8<EXACT>(qrj * M3));
    }
    // diagonal tile: fp16, bf16 hi/lo or (exact mode) fp32 operands; an
    // extreme tile is done after this loop
    if (!extreme) {
      f8 ad, bk, bqd;
#pragma unroll
      for (int e = 0; e < 8; ++e) { ad[e] = kc[j][e]; bk[e] = krj[e] * iD[e]; bqd[e] = qrj[e] * iD[e]; }
      if constexpr (EXACT) {
        accK[W] = mma32(accK[W], ad, bk);
        accQ[W] = mma32(accQ[W], ad, bqd);
      } else if (diag16) {
        const v8 a16 = cvt8<EXACT>(ad);
        accK[W] = mma32(accK[W], a16, cvt8<EXACT>(bk));
        accQ[W] = mma32(accQ[W], a16, cvt8<EXACT>(bqd));
      } else {
        // x*y ~ xh*yh + xh*yl + xl*yh with bf16 halves (x = xh + xl): ~16
        // significant bits per operand on the bf16 MFMA, with the fp32
        // exponent range the 2^|D| factor of the diagonal tile needs
        b8 ah, al, kh, kl, qh, ql;
        split_bf16(ad, ah, al);
        split_bf16(bk, kh, kl);
        split_bf16(bqd, qh, ql);
        accK[W] = mma32_bf16(accK[W], ah, kh);
        accQ[W] = mma32_bf16(accQ[W], ah, qh);
        accK[W] = mma32_bf16(accK[W], ah, kl);
        accQ[W] = mma32_bf16(accQ[W], ah, ql);
        accK[W] = mma32_bf16(accK[W], al, kh);
        accQ[W] = mma32_bf16(accQ[W], al, qh);
      }
    }

    // q*gamma -> GQ (fragment order); beta*gamma*k and lambda*k kept
    f8 gqv, lkf, bwf;
    const float bc = beta_c;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      gqv[e] = qrj[e] * P[e];
      lkf[e] = kc[j][e] * Q[e];
      bwf[e] = krj[e] * (bc * P[e]);
    }
    lk[j] = cvt8<EXACT>(lkf);
    bw[j] = cvt8<EXACT>(bwf);
    *reinterpret_cast<v8*>(oGQ + (chead * (kC / 16) * NJ + (W * NJ + j)) * 512 + l * 8) =
        cvt8<EXACT>(gqv);
  }

  // Tile decay past 2^-100 in some channel: the diagonal tile by the anchored
  // passes, K step by K step in the order the loop above would take them
  if (extreme) {
#pragma unroll 1
    for (int j = 0; j < NJ; ++j) {
      f8 acc;
#pragma unroll
      for (int i = 0; i < 4; ++i) { acc[i] = accK[W][i]; acc[4 + i] = accQ[W][i]; }
      acc = extreme_diag_step<DK, DTQ, DTG, EXACT, W, PRO>(&a, j, chead, U.len, U.row0, h, acc);
#pragma unroll
      for (int i = 0; i < 4; ++i) { accK[W][i] = acc[i]; accQ[W][i] = acc[4 + i]; }
    }
  }

  // masks; L = beta_c * Akk stays in registers (Lk[s] = 16x16x16 A fragment of L_{W,s})
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int ii = 4 * gq + i;  // key row of the tile
    if (!(r > ii)) accK[W][i] = 0.f;
    if (!(r >= ii)) accQ[W][i] = 0.f;
  }
  f4 Lk[W + 1];
#pragma unroll
  for (int s = 0; s <= W; ++s) Lk[s] = accK[s] * beta_c;
  // Aqk fragments for the state kernel: row tile W, K step jj pairs key tiles
  // (2jj, 2jj+1).  Row tiles 0 and 1 have no keys in tiles 2 and 3: their
  // jj = 1 fragment is zero, is never read, and is not stored.
#pragma unroll
  for (int jj = 0; jj < ((W < 2) ? 1 : 2); ++jj) {
    f8 x;
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      const int s = 2 * jj + hf;
#pragma unroll
      for (int i = 0; i < 4; ++i) x[4 * hf + i] = (s <= W) ? accQ[s <= W ? s : 0][i] : 0.f;
    }
    *reinterpret_cast<v8*>(oAQ + (chead * (kC / 16) * 2 + (W * 2 + jj)) * 512 + l * 8) =
        cvt8<EXACT>(x);
  }

  // lambda*k fragments for the state update, transposed by an MFMA against a
  // selection matrix: D[c][d] = sum_slot lk[c][slot] I[slot][d] lands in the D
  // layout (lane = channel d, rows c), which is half of the (lambda k)^T A
  // fragment of K step W/2.
#pragma unroll
  for (int dt = 0; dt < DK / 16; ++dt) {
    const int j = dt >> 1;
    v8 A, Isel;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      A[e] = lk[j][e];
      Isel[e] = st((gq == (r >> 2) && e == 4 * (dt & 1) + (r & 3)) ? 1.f : 0.f);
    }
    const f4 D = mma32(f4{0, 0, 0, 0}, A, Isel);
    *reinterpret_cast<v4*>(oLK + (chead * (DK / 16) * 2 + (dt * 2 + (W >> 1))) * 512 + l * 8 +
                           (W & 1) * 4) = cvt4<EXACT>(D);
  }

  // L blocks -> LDS: off-diagonal ones for the other waves' T rows, the own
  // diagonal one in fp32 for the substitution below
#pragma unroll
  for (int s = 0; s < W; ++s)
    *reinterpret_cast<v4*>(&sm.Lmb[W * (W - 1) / 2 + s][r][4 * gq]) = cvt4<EXACT>(Lk[s]);
  *reinterpret_cast<f4*>(&sm.Ld(W)[r][4 * gq]) = Lk[W];
  __builtin_amdgcn_wave_barrier();

  // diagonal block inverse: column r of T_WW by forward substitution.  The
  // L rows of four substitution steps are read from LDS together before
  // those steps (one LDS round trip per four rows, not one per row); the
  // products are summed in the same order either way.
  float x[16];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    f4 Lb[4][4];
#pragma unroll
    for (int ii = 0; ii < 4; ++ii)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        if (4 * q < 4 * b + ii) Lb[ii][q] = *reinterpret_cast<const f4*>(&sm.Ld(W)[4 * b + ii][4 * q]);
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
      const int i = 4 * b + ii;
      float acc = 0.f;
#pragma unroll
      for (int m4 = 0; m4 < i; m4 += 4) {
        const f4 Lrow = Lb[ii][m4 >> 2];
#pragma unroll
        for (int t = 0; t < 4; ++t)
          if (m4 + t < i) acc += Lrow[t] * x[m4 + t];
      }
      x[i] = (i < r) ? 0.f : ((i == r) ? 1.f : -acc);
    }
  }
  if (gq == 0) {
#pragma unroll
    for (int i = 0; i < 16; ++i) sm.Tdg[W][i][r] = st(x[i]);
  }
  lds_barrier();  // #2: Lmb, Tdg of every wave; region 1 free

  // beta*gamma*k -> region 1, channel-major (the W product's A operand)
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) sm.r1[slot_channel(j, gq, e) * PC + c] = bw[j][e];

  // rows 1..W of T in registers (each wave recomputes the earlier rows it needs):
  //   T_Rs = -T_RR sum_{j=s}^{R-1} L_Rj T_js,  T_js in the D layout (= B layout)
  f4 Toff[6];
#pragma unroll
  for (int R = 1; R <= W; ++R) {
#pragma unroll
    for (int s = R - 1; s >= 0; --s) {
      f4 X = {0, 0, 0, 0};
#pragma unroll
      for (int jb = s; jb < R; ++jb) {
        v4 A;
        if (R == W) A = cvt4<EXACT>(Lk[jb]);
        else A = *reinterpret_cast<const v4*>(&sm.Lmb[R * (R - 1) / 2 + jb][r][4 * gq]);
        v4 Bm;
        if (jb == s) {
#pragma unroll
          for (int i = 0; i < 4; ++i) Bm[i] = sm.Tdg[s][4 * gq + i][r];
        } else {
          Bm = cvt4<EXACT>(Toff[jb * (jb - 1) / 2 + s]);
        }
        X = mma16(X, A, Bm);
      }
      const v4 A2 = *reinterpret_cast<const v4*>(&sm.Tdg[R][r][4 * gq]);
      Toff[R * (R - 1) / 2 + s] = -mma16(f4{0, 0, 0, 0}, A2, cvt4<EXACT>(X));
    }
  }
  // own row block of T -> Tm (every wave reads all four after barrier #3)
#pragma unroll
  for (int s = 0; s < W; ++s)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      sm.Tm[(16 * W + 4 * gq + i) * PC + 16 * s + r] = st(Toff[W * (W - 1) / 2 + s][i]);
  if constexpr ((W & 1) == 0) {
    // the next tile's columns are inside this row's K range and must read as zero
#pragma unroll
    for (int i = 0; i < 4; ++i) sm.Tm[(16 * W + 4 * gq + i) * PC + 16 * (W + 1) + r] = st(0);
  }
  if (gq == 0) {
#pragma unroll
    for (int i = 0; i < 16; ++i) sm.Tm[(16 * W + i) * PC + 16 * W + r] = st(x[i]);
  }
  lds_barrier();  // #3: (beta*gamma*k)^T and the T row blocks of every wave

  // ---- W^T and U tiles -------------------------------------------------------
  // Balanced over the waves: wave W computes column tiles {2W, 2W+1} (of W^T's
  // dk and of U's dv) for all four row tiles, so every wave issues the same
  // 2 x (1 + 1 + 2 + 2) MFMA pairs (row tiles 0, 1 have a 32-wide K range, 2 and
  // 3 a 64-wide one) instead of the last row tile's wave doing twice the
  // first's.  A W^T pair of column tiles is one 16-byte fragment per lane.
  static_assert(DK / 16 == 8 && DV / 16 == 8 || DK / 16 == 4 && DV / 16 == 4, "column tiles per wave");
  constexpr int CT = DK / 64;          // column tiles per wave (2 at d = 128, 1 at d = 64)
  v8 Aw[CT][2], Bv[CT][2];
#pragma unroll
  for (int i = 0; i < CT; ++i)
#pragma unroll
    for (int jc = 0; jc < 2; ++jc) {
      const int t = CT * W + i;
      Aw[i][jc] = *reinterpret_cast<const v8*>(&sm.r1[(16 * t + r) * PC + 32 * jc + 8 * gq]);
      Bv[i][jc] = *reinterpret_cast<const v8*>(&sm.BVt[(16 * t + r) * PC + 32 * jc + 8 * gq]);
    }
#pragma unroll
  for (int R = 0; R < 4; ++R) {
    const int nk = (R < 2) ? 1 : 2;
    v8 Tr[2];
#pragma unroll
    for (int jc = 0; jc < 2; ++jc)
      if (jc < nk) Tr[jc] = *reinterpret_cast<const v8*>(&sm.Tm[(16 * R + r) * PC + 32 * jc + 8 * gq]);
    f4 accW[CT], accU[CT];
#pragma unroll
    for (int i = 0; i < CT; ++i) {
      accW[i] = f4{0, 0, 0, 0};
      accU[i] = f4{0, 0, 0, 0};
#pragma unroll
      for (int jc = 0; jc < 2; ++jc)
        if (jc < nk) {
          accW[i] = mma32(accW[i], Aw[i][jc], Tr[jc]);
          accU[i] = mma32(accU[i], Tr[jc], Bv[i][jc]);
        }
    }
    if constexpr (CT == 2) {
      // dk tiles 2W, 2W+1 = the two halves of K step j = W of row tile R
      v8 wf;
      const v4 w0 = cvt4<EXACT>(accW[0]), w1 = cvt4<EXACT>(accW[1]);
#pragma unroll
      for (int e = 0; e < 4; ++e) { wf[e] = w0[e]; wf[4 + e] = w1[e]; }
      *reinterpret_cast<v8*>(oW + (chead * (kC / 16) * NJ + (R * NJ + W)) * 512 + l * 8) = wf;
    } else {
      *reinterpret_cast<v4*>(oW + (chead * (kC / 16) * NJ + (R * NJ + (W >> 1))) * 512 + l * 8 +
                             (W & 1) * 4) = cvt4<EXACT>(accW[0]);
    }
#pragma unroll
    for (int i = 0; i < CT; ++i)
      *reinterpret_cast<v4*>(oU + (chead * (kC / 16) * (DV / 16) + (R * (DV / 16) + CT * W + i)) * 256 +
                             l * 4) = cvt4<EXACT>(accU[i]);
  }
}

template <int DK, int DV, bool EXACT, bool PRO, bool G32>
struct IntraLds {
  static constexpr int ROWB = DK * 2;
  static constexpr int RPI = 1024 / ROWB;
  static constexpr size_t kStage = PRO   ? static_cast<size_t>(kC + 12 * (16 + RPI)) * ROWB
                                   : G32 ? static_cast<size_t>(kC) * 4 * ROWB   // g fp32, q, k
                                         : 0;
  static constexpr size_t kBytes = sizeof(IntraSmem<DK, DV, EXACT>) > kStage ? sizeof(IntraSmem<DK, DV, EXACT>) : kStage;
};

template <int DK, int DV, int DTQ, int DTG, bool EXACT, bool PRO>
__global__ __launch_bounds__(256, EXACT ? 1 : 2)
void kda_intra_kernel(IntraArgs a) {
  __shared__ __attribute__((aligned(16))) unsigned char lds[IntraLds<DK, DV, EXACT, PRO, IntraG32<DTQ, DTG, EXACT, PRO>::value>::kBytes];
  IntraSmem<DK, DV, EXACT>& sm = *reinterpret_cast<IntraSmem<DK, DV, EXACT>*>(lds);
  const int H = a.geom.H;
  if (a.status_clear != nullptr && blockIdx.x == 0 && threadIdx.x == 0) *a.status_clear = 0;
  const int u = blockIdx.x / H;
  const int h = blockIdx.x - u * H;
  if (a.geom.cu != nullptr && a.geom.seg * a.geom.KU + u >= *a.geom.n_units) return;  // uniform per workgroup
  const UnitRef U = unit_ref(a.geom, u);
  const int64_t chead = static_cast<int64_t>(u) * H + h;
  switch (threadIdx.x >> 6) {
    case 0: intra_chunk<DK, DV, DTQ, DTG, EXACT, 0, PRO>(a, U, h, chead, sm); break;
    case 1: intra_chunk<DK, DV, DTQ, DTG, EXACT, 1, PRO>(a, U, h, chead, sm); break;
    case 2: intra_chunk<DK, DV, DTQ, DTG, EXACT, 2, PRO>(a, U, h, chead, sm); break;
    default: intra_chunk<DK, DV, DTQ, DTG, EXACT, 3, PRO>(a, U, h, chead, sm); break;
  }
}

// ----------------------------------------------------------------------------
// State step: one chunk of one chain for a 32-column value slice
// ----------------------------------------------------------------------------
template <int DK, bool EXACT>
struct StateFrags {
  typedef typename Prec<EXACT>::v8 v8;
  typedef typename Prec<EXACT>::v4 v4;
  static constexpr int NJ = DK / 32;
  static constexpr int DTW = DK / 64;
  v8 W[NJ], Q[NJ], A[2], L[DTW][2];
  v4 U[2];
  f4 gc[DTW];
};

template <int DK, int DV, bool EXACT>
struct StateSmem {
  typedef typename Prec<EXACT>::st st;
  static constexpr int PK = DK + 8;
  static constexpr int PC = kC + 8;
  st St[32 * PK];   // S^T slice: [value col][channel]
  st Vt[32 * PC];   // v~^T: [value col][row]
};

template <int DK, int DV, bool EXACT, int W>
__device__ __forceinline__ void load_frags(StateFrags<DK, EXACT>& f, const StateArgs& a,
                                           int64_t chead, int split, int l, int gq) {
  typedef typename Prec<EXACT>::st st;
  typedef typename Prec<EXACT>::v8 v8;
  typedef typename Prec<EXACT>::v4 v4;
  constexpr int NJ = DK / 32;
  constexpr int DTW = DK / 64;
  const st* iW = static_cast<const st*>(a.W);
  const st* iQ = static_cast<const st*>(a.GQ);
  const st* iA = static_cast<const st*>(a.AQ);
  const st* iL = static_cast<const st*>(a.LK);
  const st* iU = static_cast<const st*>(a.U);
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    f.W[j] = *reinterpret_cast<const v8*>(iW + (chead * (kC / 16) * NJ + (W * NJ + j)) * 512 + l * 8);
    f.Q[j] = *reinterpret_cast<const v8*>(iQ + (chead * (kC / 16) * NJ + (W * NJ + j)) * 512 + l * 8);
  }
  constexpr int NA = (W < 2) ? 1 : 2;  // Aqk row tile W has no keys past tile W
#pragma unroll
  for (int jj = 0; jj < NA; ++jj)
    f.A[jj] = *reinterpret_cast<const v8*>(iA + (chead * (kC / 16) * 2 + (W * 2 + jj)) * 512 + l * 8);
#pragma unroll
  for (int et = 0; et < 2; ++et)
    f.U[et] = *reinterpret_cast<const v4*>(
        iU + (chead * (kC / 16) * (DV / 16) + (W * (DV / 16) + 2 * split + et)) * 256 + l * 4);
#pragma unroll
  for (int t = 0; t < DTW; ++t) {
    const int dt = W * DTW + t;
#pragma unroll
    for (int jj = 0; jj < 2; ++jj)
      f.L[t][jj] = *reinterpret_cast<const v8*>(iL + (chead * (DK / 16) * 2 + (dt * 2 + jj)) * 512 + l * 8);
    f.gc[t] = *reinterpret_cast<const f4*>(a.GC + chead * DK + 16 * dt + 4 * gq);
  }
}

template <int DK, int DV, bool EXACT, int OUT_DT, int W>
__device__ __forceinline__ void state_step(f4 (&S)[DK / 64][2], const StateFrags<DK, EXACT>& f,
                                           StateSmem<DK, DV, EXACT>& sm, const StateArgs& a,
                                           int64_t row0, int len, int h, int split,
                                           int r, int gq) {
  typedef typename Prec<EXACT>::st st;
  typedef typename Prec<EXACT>::v8 v8;
  typedef typename Prec<EXACT>::v4 v4;
  constexpr int NJ = DK / 32;
  constexpr int DTW = DK / 64;
  constexpr int PK = DK + 8;
  constexpr int PC = kC + 8;
  const int H = a.geom.H;

  // 1. S^T slice -> LDS (operand precision)
#pragma unroll
  for (int t = 0; t < DTW; ++t)
#pragma unroll
    for (int et = 0; et < 2; ++et)
      *reinterpret_cast<v4*>(&sm.St[(16 * et + r) * PK + 16 * (W * DTW + t) + 4 * gq]) = cvt4<EXACT>(S[t][et]);
  lds_barrier();

  // 2. P = W S, O = (gamma q) S, v~ = U - P
  f4 O[2];
#pragma unroll
  for (int et = 0; et < 2; ++et) {
    f4 P = {0, 0, 0, 0};
    O[et] = f4{0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      v8 Sf;
      const st* row = &sm.St[(16 * et + r) * PK + 32 * j + 4 * gq];
      const v4 s0 = *reinterpret_cast<const v4*>(row);
      const v4 s1 = *reinterpret_cast<const v4*>(row + 16);
#pragma unroll
      for (int i = 0; i < 4; ++i) { Sf[i] = s0[i]; Sf[4 + i] = s1[i]; }
      P = mma32(P, f.W[j], Sf);
      O[et] = mma32(O[et], f.Q[j], Sf);
    }
    f4 vt;
#pragma unroll
    for (int i = 0; i < 4; ++i) vt[i] = static_cast<float>(f.U[et][i]) - P[i];
    *reinterpret_cast<v4*>(&sm.Vt[(16 * et + r) * PC + 16 * W + 4 * gq]) = cvt4<EXACT>(vt);
  }
  lds_barrier();

  // 3. O += Aqk v~ ; 4. S <- gamma_C S + (lambda k)^T v~
  constexpr int NA = (W < 2) ? 1 : 2;
#pragma unroll
  for (int et = 0; et < 2; ++et) {
    v8 Vf[2];
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      const st* row = &sm.Vt[(16 * et + r) * PC + 32 * jj + 4 * gq];
      const v4 s0 = *reinterpret_cast<const v4*>(row);
      const v4 s1 = *reinterpret_cast<const v4*>(row + 16);
#pragma unroll
      for (int i = 0; i < 4; ++i) { Vf[jj][i] = s0[i]; Vf[jj][4 + i] = s1[i]; }
    }
#pragma unroll
    for (int jj = 0; jj < NA; ++jj) O[et] = mma32(O[et], f.A[jj], Vf[jj]);
#pragma unroll
    for (int t = 0; t < DTW; ++t) {
      f4 s = S[t][et] * f.gc[t];
      s = mma32(s, f.L[t][0], Vf[0]);
      s = mma32(s, f.L[t][1], Vf[1]);
      S[t][et] = s;
    }
  }
  // o stores last: nothing in this step reuses their source registers, so the
  // caller's next prefetch is younger than every pending store
#pragma unroll
  for (int et = 0; et < 2; ++et)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int cr = 16 * W + 4 * gq + i;
      if (cr < len) {
        const int64_t oi = ((row0 + cr) * H + h) * (int64_t)DV + 32 * split + 16 * et + r;
        if constexpr (OUT_DT == 0) static_cast<float*>(a.o)[oi] = O[et][i];
        else static_cast<u16*>(a.o)[oi] = f32_to_bf16_bits(O[et][i]);
      }
    }
  // (the next step's first barrier orders St/Vt reuse)
}

template <int DK, int DV, bool EXACT, int OUT_DT, int W>
__device__ __forceinline__ void state_chain(const StateArgs& a, StateSmem<DK, DV, EXACT>& sm,
                                            int seq, int h, int split) {
  constexpr int DTW = DK / 64;
  const Geom& G = a.geom;
  const int H = G.H;
  const int l = threadIdx.x & 63, r = l & 15, gq = l >> 4;
  const ChainRef c = chain_ref(G, seq);
  if (!c.active) return;
  const int nchunks = c.nchunks, seq_len = c.seq_len;
  const int64_t tok0 = c.tok0;

  f4 S[DTW][2];
  const int64_t sbase = (static_cast<int64_t>(c.seq) * H + h) * DK * DV;
  const float* const s_in = c.from_h0 ? a.h0 : a.ht;
#pragma unroll
  for (int t = 0; t < DTW; ++t)
#pragma unroll
    for (int et = 0; et < 2; ++et)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = 16 * (W * DTW + t) + 4 * gq + i;
        const int e = 32 * split + 16 * et + r;
        S[t][et][i] = (s_in != nullptr) ? s_in[sbase + static_cast<int64_t>(d) * DV + e] : 0.f;
      }

  auto chead_of = [&](int n) { return static_cast<int64_t>(chain_unit(G, c, n)) * H + h; };
  auto step = [&](const StateFrags<DK, EXACT>& f, int n) {
    const int64_t row0 = tok0 + static_cast<int64_t>(n) * kC;
    const int len = min(kC, seq_len - n * kC);
    state_step<DK, DV, EXACT, OUT_DT, W>(S, f, sm, a, row0, len, h, split, r, gq);
  };
  // Three fragment sets in fixed registers.  The loads for chunk n+3 are issued
  // right after step n (and its o stores), so they are younger than every
  // store the next steps must retire before reusing registers: vmcnt retires
  // in order on this architecture, and a prefetch issued before the stores
  // would have to complete before them.
  StateFrags<DK, EXACT> f0, f1, f2;
  if (nchunks > 0) load_frags<DK, DV, EXACT, W>(f0, a, chead_of(0), split, l, gq);
  if (nchunks > 1) load_frags<DK, DV, EXACT, W>(f1, a, chead_of(1), split, l, gq);
  if (nchunks > 2) load_frags<DK, DV, EXACT, W>(f2, a, chead_of(2), split, l, gq);
  for (int n = 0; n < nchunks; n += 3) {
    step(f0, n);
    if (n + 3 < nchunks) load_frags<DK, DV, EXACT, W>(f0, a, chead_of(n + 3), split, l, gq);
    if (n + 1 >= nchunks) break;
    step(f1, n + 1);
    if (n + 4 < nchunks) load_frags<DK, DV, EXACT, W>(f1, a, chead_of(n + 4), split, l, gq);
    if (n + 2 >= nchunks) break;
    step(f2, n + 2);
    if (n + 5 < nchunks) load_frags<DK, DV, EXACT, W>(f2, a, chead_of(n + 5), split, l, gq);
  }

  if (a.ht != nullptr) {
#pragma unroll
    for (int t = 0; t < DTW; ++t)
#pragma unroll
      for (int et = 0; et < 2; ++et)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int d = 16 * (W * DTW + t) + 4 * gq + i;
          const int e = 32 * split + 16 * et + r;
          a.ht[sbase + static_cast<int64_t>(d) * DV + e] = S[t][et][i];
        }
  }
}

template <int DK, int DV, bool EXACT, int OUT_DT>
__global__ __launch_bounds__(256, 1)
void kda_state_kernel(StateArgs a) {
  constexpr int SPLITS = DV / 32;
  __shared__ StateSmem<DK, DV, EXACT> sm;
  const Geom& G = a.geom;
  const int H = G.H;
  // XCD-aware mapping: the SPLITS workgroups of one chain share an XCD (and L2)
  const int x = blockIdx.x;
  const int xcd = x & 7;
  const int kk = x >> 3;
  const int slot = kk / SPLITS;
  const int split = kk - slot * SPLITS;
  const int chain = slot * 8 + xcd;
  if (chain >= G.N * H) return;
  const int seq_rank = chain / H;
  const int h = chain - seq_rank * H;
  const int seq = seq_rank;   // the roles look the sequence up (chain_ref)
  switch (threadIdx.x >> 6) {
    case 0: state_chain<DK, DV, EXACT, OUT_DT, 0>(a, sm, seq, h, split); break;
    case 1: state_chain<DK, DV, EXACT, OUT_DT, 1>(a, sm, seq, h, split); break;
    case 2: state_chain<DK, DV, EXACT, OUT_DT, 2>(a, sm, seq, h, split); break;
    default: state_chain<DK, DV, EXACT, OUT_DT, 3>(a, sm, seq, h, split); break;
  }
}

// ----------------------------------------------------------------------------
// State kernel, column-owner form (fp16 operands)
//
// A workgroup of two waves owns 32 value columns of one chain; wave w owns
// the 16 columns of value tile et = 2*split + w for ALL dk channels, so every
// product of the step has its state / v~ operand in this wave's registers:
//   * S tile dt in the MFMA D layout (rows 4gq+i, column r) is, two tiles at a
//     time, the B fragment of a 32-wide K step over channels (slot order);
//   * v~ row tiles, two at a time, are the B fragment over 32 keys.
// Only the dv-independent A operands (W, gamma*q, Aqk, lambda*k) and gamma_C
// are shared: per chunk four producer-only waves copy them once per
// workgroup from the workspace into one of two LDS buffers (16 B per lane,
// fragment order, so every LDS read is a conflict-free 16 B per lane).  The
// copy runs two chunks ahead: a producer loads chunk n+2 into registers
// while the compute waves work on chunk n, and writes chunk n+1 (loaded one
// step earlier) into the free LDS buffer.  The compute waves issue no copies
// of their own (a wave issues memory instructions in order, so a deep copy
// queue would stall its MFMAs).  One barrier per chunk.
// ----------------------------------------------------------------------------
template <int DK>
struct ColLayout {
  static constexpr int NJ = DK / 32;
  static constexpr int FW = 4 * NJ;          // W (and gamma*q) fragments per chunk-head
  static constexpr int FL = 2 * (DK / 16);   // lambda*k fragments
  static constexpr int FA = 6;               // Aqk fragments (ct, jj) with jj <= ct / 2
  static constexpr int OFF_Q = FW;
  static constexpr int OFF_L = 2 * FW;
  static constexpr int OFF_A = 2 * FW + FL;
  static constexpr int NF = 2 * FW + FL + FA;  // 1-KiB fragments per chunk-head
  static constexpr int OFF_G = NF * 1024;      // gamma_C (DK floats)
  static constexpr int OFF_U = NF * 1024 + DK * 4;  // U of the workgroup's two value tiles, [ct][w][64][4]
  static constexpr int BYTES = OFF_U + 4 * 1024;
};

template <int DK>
struct ColSmem {
  alignas(16) unsigned char buf[2][ColLayout<DK>::BYTES];
  alignas(16) unsigned char obuf[2][kC * 32 * 4];  // o rows of the workgroup's 32 columns
};


// Producer waves per state workgroup.  One wave moves only ~22 GB/s from L2
// on this part (measured); four together move the 56 KiB a chunk needs in
// well under a chunk's compute time.
constexpr int kColProducers = 4;
// Compute waves per state workgroup; each owns 2 / kColComputeWaves of the
// workgroup's two 16-column value tiles.  (One wave owning both reads every
// shared fragment once and feeds two MFMAs; measured slower: its MFMA time
// per chunk doubles.)
constexpr int kColComputeWaves = 2;
constexpr int kColTilesPerWave = 2 / kColComputeWaves;

// Producer P's share of the o rows of one chunk: LDS [64 rows][32 columns]
// (fp32, or bf16 when OUT_DT == 1; the 16-byte chunks of rows with bit 2 set
// are swapped between the row's halves, see col_put_o) to the workgroup's 32
// columns of o, 16 B per lane, rows past the chunk's end skipped.  The stored values are kept
// in `vs` (and whether each was stored in `ok`) for the caller's range check,
// which it runs once the next chunk's copies are in flight.
template <int OUT_DT>
struct ColStoreShape {
  static constexpr int ES = (OUT_DT == 0) ? 4 : 2;
  static constexpr int LPR = 32 * ES / 16;     // lanes per row
  static constexpr int RPI = 64 / LPR;         // rows per instruction
  static constexpr int NI = kC / RPI;          // instructions per chunk
  static constexpr int NS = (NI + kColProducers - 1) / kColProducers;  // per producer
};

template <int DV, int OUT_DT, int P>
__device__ __forceinline__ void col_store_rows(const StateArgs& a, const unsigned char* ob, int64_t row0,
                                               int len, int h, int split, int l,
                                               uint4 (&vs)[ColStoreShape<OUT_DT>::NS],
                                               bool (&ok)[ColStoreShape<OUT_DT>::NS]) {
  typedef ColStoreShape<OUT_DT> SS;
  const int H = a.geom.H;
#pragma unroll
  for (int k = 0; k < SS::NS; ++k) {
    const int ins = P + kColProducers * k;
    ok[k] = false;
    vs[k] = uint4{0, 0, 0, 0};
    if (ins < SS::NI) {
      const int row = SS::RPI * ins + l / SS::LPR;
      const int cb = (l % SS::LPR) * 16;       // byte offset inside the 32-column row
      const int pcb = ((l % SS::LPR) ^ ((SS::LPR / 2) * ((row >> 2) & 1))) * 16;   // swizzled chunk
      vs[k] = *reinterpret_cast<const uint4*>(ob + row * (32 * SS::ES) + pcb);
      ok[k] = row < len;
      if (ok[k]) {
        unsigned char* dst = static_cast<unsigned char*>(a.o) +
                             (((row0 + row) * H + h) * static_cast<int64_t>(DV) + 32 * split) * SS::ES + cb;
        // non-temporal: o is not read again by this call
        __builtin_nontemporal_store(u32x4{vs[k].x, vs[k].y, vs[k].z, vs[k].w}, reinterpret_cast<u32x4*>(dst));
      }
    }
  }
}

// magnitude sum of the values col_store_rows stored
template <int OUT_DT, int NS>
__device__ __forceinline__ float col_stored_mag(const uint4 (&vs)[NS], const bool (&ok)[NS]) {
  float m = 0.f;
#pragma unroll
  for (int k = 0; k < NS; ++k) {
    const float x = (OUT_DT == 0) ? abs_sum_f32x4(vs[k]) : abs_sum_bf16x8(vs[k]);
    m += ok[k] ? x : 0.f;
  }
  return m;
}


// Calls f(std::integral_constant<int, I>{}) for I = B .. E-1, expanded at
// compile time (a loop over a long, branchy body is not always unrolled).
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// One chunk's share of producer P (every fourth shared fragment, the U block
// of row tile P for the workgroup's two value tiles, and for the last
// producer gamma_C), held in registers between its global load and its
// write into an LDS buffer.
template <int DK, int P>
struct ColRegs {
  static constexpr int NFP = (ColLayout<DK>::NF - P + kColProducers - 1) / kColProducers;
  u32x4 f[NFP];
  u32x4 u;
  u32x4 g;
};

template <int DK, int DV, int P>
__device__ __forceinline__ void col_load_regs(const StateArgs& a, int64_t ch, int split, int l,
                                              ColRegs<DK, P>& R) {
  typedef ColLayout<DK> LY;
  const _Float16* iW = static_cast<const _Float16*>(a.W);
  const _Float16* iQ = static_cast<const _Float16*>(a.GQ);
  const _Float16* iL = static_cast<const _Float16*>(a.LK);
  const _Float16* iA = static_cast<const _Float16*>(a.AQ);
  static_for<0, ColRegs<DK, P>::NFP>([&](auto kc) {
    constexpr int f = P + kColProducers * decltype(kc)::value;
    const _Float16* src;
    if constexpr (f < LY::OFF_Q) src = iW + (ch * LY::FW + f) * 512;
    else if constexpr (f < LY::OFF_L) src = iQ + (ch * LY::FW + (f - LY::OFF_Q)) * 512;
    else if constexpr (f < LY::OFF_A) src = iL + (ch * LY::FL + (f - LY::OFF_L)) * 512;
    else {
      constexpr int ai = f - LY::OFF_A;                 // 0..5 -> (ct, jj) = 00 10 20 21 30 31
      constexpr int gidx = (ai < 2) ? 2 * ai : ai + 2;  // index ct*2 + jj in the workspace
      src = iA + (ch * 8 + gidx) * 512;
    }
    R.f[decltype(kc)::value] = *reinterpret_cast<const u32x4*>(src + l * 8);
  });
  static_assert(kColProducers == 4, "one U row tile per producer");
  R.u = *reinterpret_cast<const u32x4*>(static_cast<const _Float16*>(a.U) +
                                        (ch * 4 * (DV / 16) + P * (DV / 16) + 2 * split) * 256 + l * 8);
  if constexpr (P == kColProducers - 1) {
    R.g = u32x4{0, 0, 0, 0};
    if (l < DK / 4) R.g = *reinterpret_cast<const u32x4*>(a.GC + ch * DK + l * 4);
  }
}

// The registers of one chunk into an LDS buffer, in the fragment order the
// compute waves read (lane l's 16 bytes at byte 16 l of each 1 KiB block).
template <int DK, int P>
__device__ __forceinline__ void col_write_regs(unsigned char* dst, int l, const ColRegs<DK, P>& R) {
  typedef ColLayout<DK> LY;
  static_for<0, ColRegs<DK, P>::NFP>([&](auto kc) {
    constexpr int k = decltype(kc)::value;
    *reinterpret_cast<u32x4*>(dst + (P + kColProducers * k) * 1024 + l * 16) = R.f[k];
  });
  *reinterpret_cast<u32x4*>(dst + LY::OFF_U + P * 1024 + l * 16) = R.u;
  if constexpr (P == kColProducers - 1)
    if (l < DK / 4) *reinterpret_cast<u32x4*>(dst + LY::OFF_G + l * 16) = R.g;
}

// One chunk step of producer P while the compute waves work on chunk n: store
// o of chunk n-1 (from LDS), load chunk n+2 into Rn (which held chunk n, in
// LDS since the last barrier; past the chain's end the last chunk is loaded
// again), write chunk n+1 from Rn1 into the free buffer, then join the one
// barrier per chunk.  The write waits only for Rn1's loads, issued a step
// earlier, so each load has two chunk steps to arrive.
template <int DK, int DV, int OUT_DT, int P>
__device__ __forceinline__ void col_producer_step(const StateArgs& a, ColSmem<DK>& sm, const ChainRef& c, int H,
                                                  int h, int split, int l, int n, ColRegs<DK, P>& Rn,
                                                  ColRegs<DK, P>& Rn1, float& mag) {
  constexpr int NS = ColStoreShape<OUT_DT>::NS;
  uint4 vs[NS];
  bool ok[NS];
  const bool st = n > 0;
  if (st)
    col_store_rows<DV, OUT_DT, P>(a, sm.obuf[(n - 1) & 1], c.tok0 + static_cast<int64_t>(n - 1) * kC,
                                  min(kC, c.seq_len - (n - 1) * kC), h, split, l, vs, ok);
  col_load_regs<DK, DV, P>(a, static_cast<int64_t>(chain_unit(a.geom, c, min(n + 2, c.nchunks - 1))) * H + h, split, l, Rn);
  // the range check of the stored o rows runs while the loads are in flight
  __builtin_amdgcn_sched_barrier(0);
  if (st) mag += col_stored_mag<OUT_DT>(vs, ok);
  if (n + 1 < c.nchunks) col_write_regs<DK, P>(sm.buf[(n + 1) & 1], l, Rn1);
  lds_barrier();
}

// Producer wave P of a state workgroup.  The compute waves issue no global
// memory operation inside the chunk loop: a wave issues memory instructions
// in order, so queueing behind these copies would stall their MFMAs.
template <int DK, int DV, int OUT_DT, int P>
__device__ __forceinline__ void col_producer(const StateArgs& a, ColSmem<DK>& sm, int seq, int h,
                                             int split) {
  const ChainRef c = chain_ref(a.geom, seq);
  const int H = a.geom.H;
  const int l = threadIdx.x & 63;
  if (c.nchunks <= 0) return;
  float mag = 0.f;
  const int last = c.nchunks - 1;
  ColRegs<DK, P> R0, R1;
  col_load_regs<DK, DV, P>(a, static_cast<int64_t>(chain_unit(a.geom, c, 0)) * H + h, split, l, R0);
  col_load_regs<DK, DV, P>(a, static_cast<int64_t>(chain_unit(a.geom, c, min(1, last))) * H + h, split, l, R1);
  col_write_regs<DK, P>(sm.buf[0], l, R0);
  lds_barrier();  // chunk 0 staged
  int n = 0;
  for (; n + 1 < c.nchunks; n += 2) {
    col_producer_step<DK, DV, OUT_DT, P>(a, sm, c, H, h, split, l, n, R0, R1, mag);
    col_producer_step<DK, DV, OUT_DT, P>(a, sm, c, H, h, split, l, n + 1, R1, R0, mag);
  }
  if (n < c.nchunks) col_producer_step<DK, DV, OUT_DT, P>(a, sm, c, H, h, split, l, n, R0, R1, mag);
  wait_vmem_all();
  constexpr int NS = ColStoreShape<OUT_DT>::NS;
  uint4 vs[NS];
  bool ok[NS];
  col_store_rows<DV, OUT_DT, P>(a, sm.obuf[last & 1], c.tok0 + static_cast<int64_t>(last) * kC,
                                min(kC, c.seq_len - last * kC), h, split, l, vs, ok);
  mag += col_stored_mag<OUT_DT>(vs, ok);
  report_nonfinite(a.status, mag);
}

// o of row tiles 0..3 (D layout: rows 16ct + 4gq + i, column r of value tile
// `tile` of the workgroup) into the LDS o rows of the workgroup's 32 columns.
template <int OUT_DT>
__device__ __forceinline__ void col_put_o(unsigned char* ob, const f4 (&O)[4], int tile, int r, int gq) {
#pragma unroll
  for (int ct = 0; ct < 4; ++ct)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = 16 * ct + 4 * gq + i;
      // 16-byte chunks of rows with bit 2 set swap halves, so that in each
      // 32-lane half of a write (gq 0 and 1, gq 2 and 3) the lanes hit
      // distinct banks
      constexpr int EPC = (OUT_DT == 0) ? 4 : 8;   // elements per 16-byte chunk
      const int col = 16 * tile + r;
      const int pc = ((col / EPC) ^ ((16 / EPC) * ((row >> 2) & 1))) * EPC + col % EPC;
      if constexpr (OUT_DT == 0) reinterpret_cast<float*>(ob)[row * 32 + pc] = O[ct][i];
      else reinterpret_cast<u16*>(ob)[row * 32 + pc] = f32_to_bf16_bits(O[ct][i]);
    }
}

template <int DK, int DV, int OUT_DT, int W>
__device__ __forceinline__ void col_chain(const StateArgs& a, ColSmem<DK>& sm, int seq, int h, int split) {
  typedef ColLayout<DK> LY;
  constexpr int NJ = DK / 32;
  constexpr int NT = DK / 16;
  constexpr int NC = kColTilesPerWave;
  const Geom& G = a.geom;
  const int H = G.H;
  const int l = threadIdx.x & 63, r = l & 15, gq = l >> 4;
  const int tile0 = W * NC;                 // first value tile of this wave inside the workgroup
  const ChainRef c = chain_ref(G, seq);
  if (!c.active) return;
  const int nchunks = c.nchunks;

  f4 S[NC][NT];
  const int64_t sbase = (static_cast<int64_t>(c.seq) * H + h) * DK * DV;
  const float* const s_in = c.from_h0 ? a.h0 : a.ht;
#pragma unroll
  for (int cc = 0; cc < NC; ++cc)
#pragma unroll
    for (int dt = 0; dt < NT; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        S[cc][dt][i] = (s_in != nullptr)
                           ? s_in[sbase + static_cast<int64_t>(16 * dt + 4 * gq + i) * DV +
                                  16 * (2 * split + tile0 + cc) + r]
                           : 0.f;

  if (nchunks > 0) lds_barrier();  // chunk 0 staged by the producer waves
  for (int n = 0; n < nchunks; ++n) {
    const unsigned char* cur = sm.buf[n & 1];
    h4 Ucur[NC][4];
#pragma unroll
    for (int cc = 0; cc < NC; ++cc)
#pragma unroll
      for (int ct = 0; ct < 4; ++ct)
        Ucur[cc][ct] = *reinterpret_cast<const h4*>(cur + LY::OFF_U + (2 * ct + tile0 + cc) * 512 + l * 8);

    // The step is one stream of 16-byte LDS reads consumed in order (each
    // fragment feeds one MFMA per value tile of this wave):
    //   items 0 .. 8*NJ-1    W and gamma*q fragments of K step j = i / 8, row
    //                        tile ct = (i % 8) / 2 (alternating: P and O
    //                        products), so consecutive products into one
    //                        accumulator are eight items apart (measured:
    //                        config 2 1 127 -> 1 086 us against row-tile-major
    //                        order, bit-identical),
    //   next FA items        Aqk fragments,
    //   next NT items        gamma_C of channel tile dt (one float4 per lane),
    //   last 2*NT items      lambda*k fragments, K step jj = 0 for every channel
    //                        tile dt, then K step 1.
    // Each read is issued DEPTH items ahead of its use into a register ring,
    // so up to DEPTH reads are in flight at every wait (the lgkm counter
    // tracks 15), and a scheduling barrier per item keeps that order.
    constexpr int N_ROW = 8 * NJ;
    constexpr int I_AQ = N_ROW;
    constexpr int I_GC = I_AQ + LY::FA;
    constexpr int I_LK = I_GC + NT;
    constexpr int NIT = I_LK + 2 * NT;
    constexpr int DEPTH = 12;
    constexpr int RING = DEPTH + 1;
    auto item_read = [&](auto ic) -> uint4 {
      constexpr int i = decltype(ic)::value;
      const unsigned char* p;
      if constexpr (i < N_ROW) {
        static_assert(kC == 64, "four row tiles per K step");
        constexpr int j = i / 8, ct = (i % 8) >> 1;
        p = cur + (((i & 1) ? LY::OFF_Q : 0) + ct * NJ + j) * 1024 + l * 16;
      } else if constexpr (i < I_GC) {
        p = cur + (LY::OFF_A + (i - I_AQ)) * 1024 + l * 16;
      } else if constexpr (i < I_LK) {
        p = cur + LY::OFF_G + (16 * (i - I_GC) + 4 * gq) * 4;
      } else {
        constexpr int jj = (i - I_LK) / NT, dt = (i - I_LK) % NT;
        p = cur + (LY::OFF_L + 2 * dt + jj) * 1024 + l * 16;
      }
      return *reinterpret_cast<const uint4*>(p);
    };
    uint4 ring[RING];
    static_for<0, DEPTH>([&](auto ic) { ring[decltype(ic)::value % RING] = item_read(ic); });
    // S as B fragments over channels
    h8 Sb[NC][NJ];
#pragma unroll
    for (int cc = 0; cc < NC; ++cc)
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          Sb[cc][j][i] = static_cast<_Float16>(S[cc][2 * j][i]);
          Sb[cc][j][4 + i] = static_cast<_Float16>(S[cc][2 * j + 1][i]);
        }
    f4 O[NC][4], P[NC][4], Vt[NC][4], Gc[NT];
    h8 Vb[NC][2];
#pragma unroll
    for (int cc = 0; cc < NC; ++cc)
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) { P[cc][ct] = f4{0, 0, 0, 0}; O[cc][ct] = f4{0, 0, 0, 0}; }
    static_for<0, NIT>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      if constexpr (i + DEPTH < NIT) ring[(i + DEPTH) % RING] = item_read(std::integral_constant<int, i + DEPTH>{});
      __builtin_amdgcn_sched_barrier(0);
      const uint4 it = ring[i % RING];
      if constexpr (i < N_ROW) {
        // P = W S and O = (gamma q) S, K step j of row tile ct; v~ = U - P
        // once every P is complete
        constexpr int j = i / 8, ct = (i % 8) >> 1;
        const h8 A = __builtin_bit_cast(h8, it);
#pragma unroll
        for (int cc = 0; cc < NC; ++cc) {
          if constexpr (i & 1) O[cc][ct] = mma32(O[cc][ct], A, Sb[cc][j]);
          else P[cc][ct] = mma32(P[cc][ct], A, Sb[cc][j]);
        }
        if constexpr (i == N_ROW - 1) {
#pragma unroll
          for (int cc = 0; cc < NC; ++cc)
#pragma unroll
            for (int t4 = 0; t4 < 4; ++t4)
#pragma unroll
              for (int e = 0; e < 4; ++e) Vt[cc][t4][e] = static_cast<float>(Ucur[cc][t4][e]) - P[cc][t4][e];
        }
      } else if constexpr (i < I_GC) {
        // O += Aqk v~ (keys at or before the row tile); fragments (ct,jj) = 00 10 20 21 30 31
        constexpr int f = i - I_AQ;
        if constexpr (f == 0) {
#pragma unroll
          for (int cc = 0; cc < NC; ++cc)
#pragma unroll
            for (int jj = 0; jj < 2; ++jj)
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                Vb[cc][jj][e] = static_cast<_Float16>(Vt[cc][2 * jj][e]);
                Vb[cc][jj][4 + e] = static_cast<_Float16>(Vt[cc][2 * jj + 1][e]);
              }
        }
        constexpr int ct = (f < 2) ? f : 2 + ((f - 2) >> 1);
        constexpr int jj = (f < 2) ? 0 : ((f - 2) & 1);
        const h8 A = __builtin_bit_cast(h8, it);
#pragma unroll
        for (int cc = 0; cc < NC; ++cc) O[cc][ct] = mma32(O[cc][ct], A, Vb[cc][jj]);
      } else if constexpr (i < I_LK) {
        Gc[i - I_GC] = __builtin_bit_cast(f4, it);
      } else {
        // S <- gamma_C S + (lambda k)^T v~, K step jj of channel tile dt
        constexpr int jj = (i - I_LK) / NT, dt = (i - I_LK) % NT;
        const h8 A = __builtin_bit_cast(h8, it);
#pragma unroll
        for (int cc = 0; cc < NC; ++cc) {
          if constexpr (jj == 0) S[cc][dt] = S[cc][dt] * Gc[dt];
          S[cc][dt] = mma32(S[cc][dt], A, Vb[cc][jj]);
        }
      }
    });

#pragma unroll
    for (int cc = 0; cc < NC; ++cc) col_put_o<OUT_DT>(sm.obuf[n & 1], O[cc], tile0 + cc, r, gq);
    // the producers have landed the next buffer and may store these o rows;
    // the compute waves are done with this buffer before it is refilled
    lds_barrier();
  }

  if (a.ht != nullptr) {
    float mag = 0.f;
#pragma unroll
    for (int cc = 0; cc < NC; ++cc)
#pragma unroll
      for (int dt = 0; dt < NT; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          mag += fabsf(S[cc][dt][i]);
          a.ht[sbase + static_cast<int64_t>(16 * dt + 4 * gq + i) * DV + 16 * (2 * split + tile0 + cc) + r] =
              S[cc][dt][i];
        }
    report_nonfinite(a.status, mag);
  }
}

template <int DK, int DV, int OUT_DT>
__global__ __launch_bounds__(64 * (kColComputeWaves + kColProducers), 1)
void kda_state_col_kernel(StateArgs a) {
  constexpr int SPLITS = DV / 32;
  __shared__ ColSmem<DK> sm;
  const Geom& G = a.geom;
  const int H = G.H;
  // XCD-aware mapping: the SPLITS workgroups of one chain share an XCD (and L2)
  const int x = blockIdx.x;
  const int xcd = x & 7;
  const int kk = x >> 3;
  const int slot = kk / SPLITS;
  const int split = kk - slot * SPLITS;
  const int chain = slot * 8 + xcd;
  if (chain >= G.N * H) return;
  const int seq_rank = chain / H;
  const int h = chain - seq_rank * H;
  const int seq = seq_rank;   // the roles look the sequence up (chain_ref)
  const int wave = threadIdx.x >> 6;
  if (wave < kColComputeWaves) {
    if constexpr (kColComputeWaves == 1) col_chain<DK, DV, OUT_DT, 0>(a, sm, seq, h, split);
    else if (wave == 0) col_chain<DK, DV, OUT_DT, 0>(a, sm, seq, h, split);
    else col_chain<DK, DV, OUT_DT, 1>(a, sm, seq, h, split);
  } else {
    switch (wave - kColComputeWaves) {
      case 0: col_producer<DK, DV, OUT_DT, 0>(a, sm, seq, h, split); break;
      case 1: col_producer<DK, DV, OUT_DT, 1>(a, sm, seq, h, split); break;
      case 2: col_producer<DK, DV, OUT_DT, 2>(a, sm, seq, h, split); break;
      default: col_producer<DK, DV, OUT_DT, 3>(a, sm, seq, h, split); break;
    }
  }
}

// ----------------------------------------------------------------------------
// State kernel, wide-slice form (fp16 operands)
//
// A workgroup owns VT value tiles (16 columns each) of one chain: compute
// wave w owns VT / CW of them for all dk channels, so every shared fragment
// it reads from LDS feeds one MFMA per value tile it owns; four producer
// waves copy the chunk's shared operands, gamma_C and the workgroup's U into
// one of two LDS buffers one chunk ahead.  The compute waves store o straight
// from their accumulators: they issue no loads, so their stores queue behind
// nothing.  Against the 32-column form, the shared operands of a chunk are
// copied into LDS once per VT value tiles instead of once per two, and each
// LDS read feeds more MFMA work; the serial step is longer.  VT = 8 (the
// whole chain) pays when the chains fill the CUs, VT = 4 in between.
// ----------------------------------------------------------------------------
template <int DK, int VT>
struct WideLayout {
  typedef ColLayout<DK> CL;
  static constexpr int NF = CL::NF;
  static constexpr int OFF_G = NF * 1024;                       // gamma_C (DK floats)
  static constexpr int OFF_U = NF * 1024 + DK * 4;              // U [ct][VT][64][4] fp16
  static constexpr int BYTES = OFF_U + 4 * VT * 512;
};

template <int DK, int VT>
struct WideSmem {
  alignas(16) unsigned char buf[2][WideLayout<DK, VT>::BYTES];
};

constexpr int kWideProducers = 4;

// Producer P's share of chunk-head ch: every fourth shared fragment, U row
// tile P of the workgroup's value tiles, and (last producer) gamma_C.  The
// copies are non-temporal: one workgroup owns the whole chain, so no other
// workgroup reads these lines (config 3 3 990 -> 3 930 us when introduced).
template <int DK, int DV, int VT, int P>
__device__ __forceinline__ void wide_stage(const StateArgs& a, int64_t ch, int split, unsigned char* dst, int l) {
  typedef ColLayout<DK> LY;
  typedef WideLayout<DK, VT> WL;
  const _Float16* iW = static_cast<const _Float16*>(a.W);
  const _Float16* iQ = static_cast<const _Float16*>(a.GQ);
  const _Float16* iL = static_cast<const _Float16*>(a.LK);
  const _Float16* iA = static_cast<const _Float16*>(a.AQ);
#pragma unroll
  for (int f = P; f < LY::NF; f += kWideProducers) {
    const _Float16* src;
    if (f < LY::OFF_Q) src = iW + (ch * LY::FW + f) * 512;
    else if (f < LY::OFF_L) src = iQ + (ch * LY::FW + (f - LY::OFF_Q)) * 512;
    else if (f < LY::OFF_A) src = iL + (ch * LY::FL + (f - LY::OFF_L)) * 512;
    else {
      const int ai = f - LY::OFF_A;                 // 0..5 -> (ct, jj) = 00 10 20 21 30 31
      const int gidx = (ai < 2) ? 2 * ai : ai + 2;  // index ct*2 + jj in the workspace
      src = iA + (ch * 8 + gidx) * 512;
    }
    __builtin_amdgcn_global_load_lds(src + l * 8, dst + f * 1024, 16, 0, kCpolStream);
  }
  static_assert(kWideProducers == 4, "one U row tile per producer");
#pragma unroll
  for (int i = 0; i < VT / 2; ++i) {
    // value tiles 2i, 2i+1 of the workgroup, row tile P: 1 KiB, contiguous in the workspace
    const _Float16* usrc = static_cast<const _Float16*>(a.U) +
                           (ch * 4 * (DV / 16) + P * (DV / 16) + split * VT + 2 * i) * 256 + l * 8;
    __builtin_amdgcn_global_load_lds(usrc, dst + WL::OFF_U + (P * VT + 2 * i) * 512, 16, 0, kCpolStream);
  }
  if constexpr (P == kWideProducers - 1) {
    const _Float16* gsrc = reinterpret_cast<const _Float16*>(a.GC + ch * DK + l * 4);
    if (l < DK / 4) __builtin_amdgcn_global_load_lds(gsrc, dst + WL::OFF_G, 16, 0, kCpolStream);
  }
}

template <int DK, int DV, int VT, int P>
__device__ __forceinline__ void wide_producer(const StateArgs& a, WideSmem<DK, VT>& sm, int seq, int h, int split) {
  const ChainRef c = chain_ref(a.geom, seq);
  const int H = a.geom.H;
  const int l = threadIdx.x & 63;
  if (c.nchunks <= 0) return;
  wide_stage<DK, DV, VT, P>(a, static_cast<int64_t>(chain_unit(a.geom, c, 0)) * H + h, split, sm.buf[0], l);
  wait_vmem_all();
  lds_barrier();
  for (int n = 0; n < c.nchunks; ++n) {
    if (n + 1 < c.nchunks)
      wide_stage<DK, DV, VT, P>(a, static_cast<int64_t>(chain_unit(a.geom, c, n + 1)) * H + h, split,
                                sm.buf[(n + 1) & 1], l);
    wait_vmem_all();
    lds_barrier();
  }
}

template <int DK, int DV, int VT, int CW, int OUT_DT, int W>
__device__ __forceinline__ void wide_chain(const StateArgs& a, WideSmem<DK, VT>& sm, int seq, int h, int split) {
  typedef ColLayout<DK> LY;
  typedef WideLayout<DK, VT> WL;
  constexpr int NJ = DK / 32;
  constexpr int NT = DK / 16;
  constexpr int NC = VT / CW;                   // value tiles of this wave
  const Geom& G = a.geom;
  const int H = G.H;
  const int l = threadIdx.x & 63, r = l & 15, gq = l >> 4;
  const int tile0 = W * NC;                     // first value tile of this wave inside the workgroup
  const int col0 = 16 * (split * VT + tile0);   // its first value column in the chain
  const ChainRef c = chain_ref(G, seq);
  if (!c.active) return;
  const int nchunks = c.nchunks;

  f4 S[NC][NT];
  const int64_t sbase = (static_cast<int64_t>(c.seq) * H + h) * DK * DV;
  const float* const s_in = c.from_h0 ? a.h0 : a.ht;
#pragma unroll
  for (int cc = 0; cc < NC; ++cc)
#pragma unroll
    for (int dt = 0; dt < NT; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        S[cc][dt][i] = (s_in != nullptr)
                           ? s_in[sbase + static_cast<int64_t>(16 * dt + 4 * gq + i) * DV + col0 + 16 * cc + r]
                           : 0.f;

  float mag = 0.f;
  if (nchunks > 0) lds_barrier();  // chunk 0 staged by the producer waves
  for (int n = 0; n < nchunks; ++n) {
    const unsigned char* cur = sm.buf[n & 1];
    // Item stream of the step, 16-byte LDS reads consumed in order (each
    // fragment feeds one MFMA per value tile of this wave):
    //   items 0 .. 8*NJ-1   W and gamma*q fragments of row tile ct = i / (2*NJ)
    //                       (alternating: the P and O products of K step j),
    //   next FA items       Aqk fragments,
    //   last 3*NT items     per channel tile dt: gamma_C (one float4 per
    //                       lane), then the lambda*k fragments of K steps 0, 1.
    constexpr int N_ROW = 8 * NJ;
    constexpr int I_AQ = N_ROW;
    constexpr int I_LK = I_AQ + LY::FA;
    constexpr int NIT = I_LK + 3 * NT;
    constexpr int DEPTH = 6;
    constexpr int RING = DEPTH + 1;
    auto item_read = [&](auto ic) -> uint4 {
      constexpr int i = decltype(ic)::value;
      const unsigned char* p;
      if constexpr (i < N_ROW) {
        constexpr int ct = i / (2 * NJ), j = (i % (2 * NJ)) >> 1;
        p = cur + (((i & 1) ? LY::OFF_Q : 0) + ct * NJ + j) * 1024 + l * 16;
      } else if constexpr (i < I_LK) {
        p = cur + (LY::OFF_A + (i - I_AQ)) * 1024 + l * 16;
      } else {
        constexpr int dt = (i - I_LK) / 3, k3 = (i - I_LK) % 3;
        if constexpr (k3 == 0) p = cur + WL::OFF_G + (16 * dt + 4 * gq) * 4;
        else p = cur + (LY::OFF_L + 2 * dt + (k3 - 1)) * 1024 + l * 16;
      }
      return *reinterpret_cast<const uint4*>(p);
    };
    uint4 ring[RING];
    static_for<0, DEPTH>([&](auto ic) { ring[decltype(ic)::value % RING] = item_read(ic); });
    h4 Ucur[NC][4];
#pragma unroll
    for (int cc = 0; cc < NC; ++cc)
#pragma unroll
      for (int ct = 0; ct < 4; ++ct)
        Ucur[cc][ct] = *reinterpret_cast<const h4*>(cur + WL::OFF_U + (ct * VT + tile0 + cc) * 512 + l * 8);
    // S as B fragments over channels
    h8 Sb[NC][NJ];
#pragma unroll
    for (int cc = 0; cc < NC; ++cc)
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          Sb[cc][j][i] = static_cast<_Float16>(S[cc][2 * j][i]);
          Sb[cc][j][4 + i] = static_cast<_Float16>(S[cc][2 * j + 1][i]);
        }
    f4 O[NC][4], P[NC], Gc;
    h4 Vh[NC][4];
    h8 Vb[NC][2];
#pragma unroll
    for (int cc = 0; cc < NC; ++cc)
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) O[cc][ct] = f4{0, 0, 0, 0};
    static_for<0, NIT>([&](auto ic) {
      constexpr int i = decltype(ic)::value;
      if constexpr (i + DEPTH < NIT) ring[(i + DEPTH) % RING] = item_read(std::integral_constant<int, i + DEPTH>{});
      __builtin_amdgcn_sched_barrier(0);
      const uint4 it = ring[i % RING];
      if constexpr (i < N_ROW) {
        // P = W S and O = (gamma q) S, row tile ct; v~ = U - P once P is complete
        constexpr int ct = i / (2 * NJ), j = (i % (2 * NJ)) >> 1;
        const h8 A = __builtin_bit_cast(h8, it);
#pragma unroll
        for (int cc = 0; cc < NC; ++cc) {
          if constexpr (i & 1) {
            O[cc][ct] = mma32(O[cc][ct], A, Sb[cc][j]);
          } else {
            if constexpr (j == 0) P[cc] = mma32(f4{0, 0, 0, 0}, A, Sb[cc][j]);
            else P[cc] = mma32(P[cc], A, Sb[cc][j]);
          }
        }
        if constexpr (i % (2 * NJ) == 2 * NJ - 1) {
#pragma unroll
          for (int cc = 0; cc < NC; ++cc)
#pragma unroll
            for (int e = 0; e < 4; ++e)
              Vh[cc][ct][e] = static_cast<_Float16>(static_cast<float>(Ucur[cc][ct][e]) - P[cc][e]);
        }
      } else if constexpr (i < I_LK) {
        // O += Aqk v~ (keys at or before the row tile); fragments (ct,jj) = 00 10 20 21 30 31
        constexpr int f = i - I_AQ;
        if constexpr (f == 0) {
#pragma unroll
          for (int cc = 0; cc < NC; ++cc)
#pragma unroll
            for (int jj = 0; jj < 2; ++jj)
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                Vb[cc][jj][e] = Vh[cc][2 * jj][e];
                Vb[cc][jj][4 + e] = Vh[cc][2 * jj + 1][e];
              }
        }
        constexpr int ct = (f < 2) ? f : 2 + ((f - 2) >> 1);
        constexpr int jj = (f < 2) ? 0 : ((f - 2) & 1);
        const h8 A = __builtin_bit_cast(h8, it);
#pragma unroll
        for (int cc = 0; cc < NC; ++cc) O[cc][ct] = mma32(O[cc][ct], A, Vb[cc][jj]);
      } else {
        // S <- gamma_C S + (lambda k)^T v~ for channel tile dt
        constexpr int dt = (i - I_LK) / 3, k3 = (i - I_LK) % 3;
        if constexpr (k3 == 0) {
          Gc = __builtin_bit_cast(f4, it);
        } else {
          const h8 A = __builtin_bit_cast(h8, it);
#pragma unroll
          for (int cc = 0; cc < NC; ++cc) {
            if constexpr (k3 == 1) S[cc][dt] = S[cc][dt] * Gc;
            S[cc][dt] = mma32(S[cc][dt], A, Vb[cc][k3 - 1]);
          }
        }
      }
    });

    // o of this chunk straight from the accumulators (rows past the end skipped)
    const int64_t row0 = c.tok0 + static_cast<int64_t>(n) * kC;
    const int len = min(kC, c.seq_len - n * kC);
#pragma unroll
    for (int cc = 0; cc < NC; ++cc)
#pragma unroll
      for (int ct = 0; ct < 4; ++ct)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int row = 16 * ct + 4 * gq + i;
          if (row < len) {
            const int64_t oi = ((row0 + row) * H + h) * static_cast<int64_t>(DV) + col0 + 16 * cc + r;
            mag += fabsf(O[cc][ct][i]);
            if constexpr (OUT_DT == 0) static_cast<float*>(a.o)[oi] = O[cc][ct][i];
            else static_cast<u16*>(a.o)[oi] = f32_to_bf16_bits(O[cc][ct][i]);
          }
        }
    // the producers have landed the next buffer; this one is refilled only
    // after every compute wave has passed this barrier
    lds_barrier();
  }

  if (a.ht != nullptr) {
#pragma unroll
    for (int cc = 0; cc < NC; ++cc)
#pragma unroll
      for (int dt = 0; dt < NT; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          mag += fabsf(S[cc][dt][i]);
          a.ht[sbase + static_cast<int64_t>(16 * dt + 4 * gq + i) * DV + col0 + 16 * cc + r] = S[cc][dt][i];
        }
  }
  report_nonfinite(a.status, mag);
}

template <int DK, int DV, int VT, int CW, int OUT_DT>
__global__ __launch_bounds__(64 * (CW + kWideProducers), 1)
void kda_state_wide_kernel(StateArgs a) {
  constexpr int SPL = DV / 16 / VT;   // workgroups per chain
  __shared__ WideSmem<DK, VT> sm;
  const Geom& G = a.geom;
  const int H = G.H;
  // XCD-aware mapping: the SPL workgroups of one chain share an XCD (and L2)
  const int x = blockIdx.x;
  const int xcd = x & 7;
  const int kk = x >> 3;
  const int slot = kk / SPL;
  const int split = kk - slot * SPL;
  const int chain = slot * 8 + xcd;
  if (chain >= G.N * H) return;
  const int seq_rank = chain / H;
  const int h = chain - seq_rank * H;
  const int seq = seq_rank;   // the roles look the sequence up (chain_ref)
  const int wave = threadIdx.x >> 6;
  if (wave < CW) {
    static_for<0, CW>([&](auto wc) {
      if (wave == decltype(wc)::value) wide_chain<DK, DV, VT, CW, OUT_DT, decltype(wc)::value>(a, sm, seq, h, split);
    });
  } else {
    switch (wave - CW) {
      case 0: wide_producer<DK, DV, VT, 0>(a, sm, seq, h, split); break;
      case 1: wide_producer<DK, DV, VT, 1>(a, sm, seq, h, split); break;
      case 2: wide_producer<DK, DV, VT, 2>(a, sm, seq, h, split); break;
      default: wide_producer<DK, DV, VT, 3>(a, sm, seq, h, split); break;
    }
  }
}

// ----------------------------------------------------------------------------
// Overlapped segments: the state scan of segment s and the intra-chunk work
// of segment s+1 in one launch (fp16 operands).
//
// With few chains the 32-column state workgroups occupy few CUs (one each:
// 133 KiB of LDS) and the serial chain leaves the rest of the chip idle.
// Workgroups below `n_state` take the state role (kda_state_col_kernel's
// mapping; they are dispatched first and land one per CU); the others take
// two chunk-heads of the next segment each (waves 0-3 and 4-7, one
// IntraSmem each, in step: both run the same barriers).  The two segments use
// different halves of a double workspace, so no workgroup waits for another.
// ----------------------------------------------------------------------------
// barriers of intra_chunk on the staged 16-bit path: the staging barrier and #1-#3
constexpr int kIntraBarriers = 4;

template <int DK, int DV, bool G32>
struct OverlapLds {
  static constexpr size_t kIntra = 2 * IntraLds<DK, DV, false, false, G32>::kBytes;
  static constexpr size_t kState = sizeof(ColSmem<DK>);
  static constexpr size_t kBytes = kIntra > kState ? kIntra : kState;
};

template <int DK, int DV, int DTQ, int DTG, int OUT_DT>
__global__ __launch_bounds__(512, 1)
void kda_overlap_kernel(IntraArgs ia, StateArgs sa, int n_state) {
  constexpr bool G32 = IntraG32<DTQ, DTG, false, false>::value;
  __shared__ __attribute__((aligned(16))) unsigned char lds[OverlapLds<DK, DV, G32>::kBytes];
  const int wave = threadIdx.x >> 6;
  if (static_cast<int>(blockIdx.x) < n_state) {
    constexpr int SPLITS = DV / 32;
    ColSmem<DK>& sm = *reinterpret_cast<ColSmem<DK>*>(lds);
    const Geom& G = sa.geom;
    const int H = G.H;
    const int x = blockIdx.x;
    const int xcd = x & 7;
    const int kk = x >> 3;
    const int slot = kk / SPLITS;
    const int split = kk - slot * SPLITS;
    const int chain = slot * 8 + xcd;
    if (chain >= G.N * H) return;  // uniform per workgroup
    const int seq_rank = chain / H;
    const int h = chain - seq_rank * H;
    const int seq = seq_rank;   // the roles look the sequence up (chain_ref)
    static_assert(kColComputeWaves == 2 && kColProducers == 4, "six working waves");
    switch (wave) {
      case 0: col_chain<DK, DV, OUT_DT, 0>(sa, sm, seq, h, split); break;
      case 1: col_chain<DK, DV, OUT_DT, 1>(sa, sm, seq, h, split); break;
      case 2: col_producer<DK, DV, OUT_DT, 0>(sa, sm, seq, h, split); break;
      case 3: col_producer<DK, DV, OUT_DT, 1>(sa, sm, seq, h, split); break;
      case 4: col_producer<DK, DV, OUT_DT, 2>(sa, sm, seq, h, split); break;
      case 5: col_producer<DK, DV, OUT_DT, 3>(sa, sm, seq, h, split); break;
      default: {
        // the two spare waves join every barrier of the state role
        const int nb = chain_ref(G, seq).nchunks;
        for (int i = 0; i < (nb > 0 ? nb + 1 : 0); ++i) lds_barrier();
        break;
      }
    }
  } else {
    const int grp = wave >> 2;
    IntraSmem<DK, DV, false>& sm =
        *reinterpret_cast<IntraSmem<DK, DV, false>*>(lds + grp * IntraLds<DK, DV, false, false, G32>::kBytes);
    const int H = ia.geom.H;
    const int x = 2 * (static_cast<int>(blockIdx.x) - n_state) + grp;
    if (x < ia.total) {
      const int u = x / H;
      const int h = x - u * H;
      const UnitRef U = unit_ref(ia.geom, u);
      const int64_t chead = static_cast<int64_t>(u) * H + h;
      switch (wave & 3) {
        case 0: intra_chunk<DK, DV, DTQ, DTG, false, 0, false>(ia, U, h, chead, sm); break;
        case 1: intra_chunk<DK, DV, DTQ, DTG, false, 1, false>(ia, U, h, chead, sm); break;
        case 2: intra_chunk<DK, DV, DTQ, DTG, false, 2, false>(ia, U, h, chead, sm); break;
        default: intra_chunk<DK, DV, DTQ, DTG, false, 3, false>(ia, U, h, chead, sm); break;
      }
    } else {
      // no chunk-head for this group: join the other group's barriers
      for (int i = 0; i < kIntraBarriers; ++i) lds_barrier();
    }
  }
}

// ----------------------------------------------------------------------------
// host-side launchers
// ----------------------------------------------------------------------------
template <int DK, int DV, int DTQ, int DTG, bool EXACT, bool PRO = false>
static hipError_t launch_intra_t(const IntraArgs& a, int grid, hipStream_t s) {
  hipLaunchKernelGGL((kda_intra_kernel<DK, DV, DTQ, DTG, EXACT, PRO>), dim3(grid), dim3(256), 0, s, a);
  return hipGetLastError();
}

// The whole-chain state kernel (VT = 8) runs a chunk step in ~2.3 us against
// ~1.4 us for the 32-column slices, with four times the work per CU: it pays
// when there are enough chains to fill the CUs (config 3, 1 024 chains:
// 4 575 -> 4 025 us per call), and the 32-column slices pay when the serial
// chain is the critical path.  64-column slices (VT = 4, two compute waves of
// two value tiles) lost at every measured shape (config 1 229 -> 277 us,
// config 2 1 569 -> 2 465 us), so calls with fewer chains keep the 32-column
// slices.
constexpr int kFullStateMinChains = 256;
template <int DK, int DV, bool EXACT, int OUT>
static hipError_t launch_state_t(const StateArgs& a, int grid, hipStream_t s) {
  if constexpr (EXACT) {
    hipLaunchKernelGGL((kda_state_kernel<DK, DV, EXACT, OUT>), dim3(grid), dim3(256), 0, s, a);
  } else {
    const int64_t chains = static_cast<int64_t>(a.geom.N) * a.geom.H;
    if (DK == 128 && chains >= kFullStateMinChains) {
      hipLaunchKernelGGL((kda_state_wide_kernel<DK, DV, DV / 16, 4, OUT>), dim3(((chains + 7) / 8) * 8),
                         dim3(64 * (4 + kWideProducers)), 0, s, a);
    } else {
      hipLaunchKernelGGL((kda_state_col_kernel<DK, DV, OUT>), dim3(grid), dim3(64 * (kColComputeWaves + kColProducers)), 0,
                         s, a);
    }
  }
  return hipGetLastError();
}

hipError_t launch_intra(const IntraArgs& a, int d, int dtq, int dtg, int grid, hipStream_t s) {
#define KDA_INTRA(D, Q, G, E) \
  if (d == D && dtq == Q && dtg == G) return launch_intra_t<D, D, Q, G, E>(a, grid, s);
  KDA_INTRA(128, 1, 1, false)
  KDA_INTRA(128, 2, 2, false)
  KDA_INTRA(128, 1, 0, false)
  KDA_INTRA(128, 0, 0, true)
  KDA_INTRA(64, 1, 1, false)
  KDA_INTRA(64, 2, 2, false)
  KDA_INTRA(64, 1, 0, false)
  KDA_INTRA(64, 0, 0, true)
#undef KDA_INTRA
  return hipErrorInvalidValue;
}

hipError_t launch_intra_prologue(const IntraArgs& a, int d, int dtg, int grid, hipStream_t s) {
  if (a.K < 1 || a.K > kFusedConvTaps) return hipErrorInvalidValue;
  if (d == 128 && dtg == 1) return launch_intra_t<128, 128, 1, 1, false, true>(a, grid, s);
  if (d == 128 && dtg == 0) return launch_intra_t<128, 128, 1, 0, false, true>(a, grid, s);
  if (d == 64 && dtg == 1) return launch_intra_t<64, 64, 1, 1, false, true>(a, grid, s);
  if (d == 64 && dtg == 0) return launch_intra_t<64, 64, 1, 0, false, true>(a, grid, s);
  return hipErrorInvalidValue;
}

// One launch: the state role for segment s (n_state workgroups, the 32-column
// state kernel's grid) and the intra role for segment s+1 (ia.total
// chunk-heads, two per workgroup).
hipError_t launch_overlap(const IntraArgs& ia0, const StateArgs& sa, int d, int dtq, int dtg, int out_dt,
                          int n_state, int intra_units, hipStream_t s) {
  IntraArgs ia = ia0;
  ia.total = intra_units;
  const int grid = n_state + (intra_units + 1) / 2;
#define KDA_OVL(D, Q, G, O)                                                                            \
  if (d == D && dtq == Q && dtg == G && out_dt == O) {                                                 \
    hipLaunchKernelGGL((kda_overlap_kernel<D, D, Q, G, O>), dim3(grid), dim3(512), 0, s, ia, sa, n_state); \
    return hipGetLastError();                                                                          \
  }
  KDA_OVL(128, 1, 1, 0)
  KDA_OVL(128, 1, 1, 1)
  KDA_OVL(128, 2, 2, 0)
  KDA_OVL(128, 2, 2, 1)
  KDA_OVL(128, 1, 0, 0)
  KDA_OVL(128, 1, 0, 1)
  KDA_OVL(64, 1, 1, 0)
  KDA_OVL(64, 1, 1, 1)
  KDA_OVL(64, 2, 2, 0)
  KDA_OVL(64, 2, 2, 1)
  KDA_OVL(64, 1, 0, 0)
  KDA_OVL(64, 1, 0, 1)
#undef KDA_OVL
  return hipErrorInvalidValue;
}

hipError_t launch_state(const StateArgs& a, int d, bool exact, int out_dt, int grid, hipStream_t s) {
#define KDA_STATE(D, E, O) \
  if (d == D && exact == E && out_dt == O) return launch_state_t<D, D, E, O>(a, grid, s);
  KDA_STATE(128, false, 0)
  KDA_STATE(128, false, 1)
  KDA_STATE(128, true, 0)
  KDA_STATE(128, true, 1)
  KDA_STATE(64, false, 0)
  KDA_STATE(64, false, 1)
  KDA_STATE(64, true, 0)
  KDA_STATE(64, true, 1)
#undef KDA_STATE
  return hipErrorInvalidValue;
}

}  // namespace kda
