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
// Two kernels:
//  * kda_intra_kernel  -- one workgroup per chunk-head, fully parallel.  Builds
//    the decay-gated scores on MFMA (off-diagonal 16x16 tiles with both decay
//    factors <= 1 in fp16; diagonal tiles with a mid-tile anchor in a bf16
//    hi/lo split, 3 MFMAs, ~fp32 accuracy), solves T = (I+L)^-1 in LDS
//    (column substitution for the 16x16 diagonal blocks, MFMA for the
//    off-diagonal blocks), forms W and U, and writes W, U, Aqk, gamma*q,
//    lambda*k and gamma_C to the workspace in MFMA fragment order.
//  * kda_state_kernel  -- one workgroup per (chain, 32-column dv slice); walks
//    the chunks of its chain in order with the fp32 state slice S[dk x 32]
//    held in MFMA accumulators, and emits o.
//
// Exact mode (fp32 inputs) uses the same code with fp32 operands and
// 16x16x4 fp32 MFMAs.

#include "kda_common.h"
#include "kda_internal.h"

namespace kda {

constexpr int kC = 64;

// ----------------------------------------------------------------------------
// chunk-unit geometry
// ----------------------------------------------------------------------------
struct UnitRef {
  int seq;        // sequence (dense: batch index)
  int n;          // chunk index inside the sequence
  int64_t row0;   // first token (global token index into [B*T] or the packed T)
  int len;        // valid rows, 1..64
};

__device__ __forceinline__ UnitRef unit_ref(const Geom& G, int u) {
  UnitRef R;
  if (G.cu == nullptr) {
    R.seq = u / G.NT;
    R.n = u - R.seq * G.NT;
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

// ----------------------------------------------------------------------------
// Intra-chunk kernel
// ----------------------------------------------------------------------------
template <int DK, int DV, bool EXACT>
struct IntraSmem {
  typedef typename Prec<EXACT>::st st;
  static constexpr int PK = DK + 8;   // row pitch (elements) of [C][DK] buffers
  static constexpr int PC = kC + 8;   // row pitch of [*][C] buffers
  st KC[kC * PK];         // k*Cf (slot order); later the lambda*k transpose stage
  st BWt[DK * PC];        // (beta*gamma*k)^T, rows = channel
  st BVt[DV * PC];        // (beta*v)^T
  st Lm[kC * PC];         // L (off-diagonal blocks)
  st Tm[kC * PC];         // T = (I+L)^-1
  float Ld[4][16][17];    // diagonal blocks of L, fp32
  float tot[4][DK];       // per-tile log2 decay totals, slot order
  float beta_s[kC];
};

template <int DK, int DV, int DTQ, int DTG, bool EXACT>
__global__ __launch_bounds__(256, EXACT ? 1 : 2)
void kda_intra_kernel(IntraArgs a) {
  typedef typename Prec<EXACT>::st st;
  typedef typename Prec<EXACT>::v8 v8;
  typedef typename Prec<EXACT>::v4 v4;
  typedef IntraSmem<DK, DV, EXACT> SM;
  constexpr int NJ = DK / 32;     // 32-wide K steps over dk
  constexpr int NJV = DV / 32;
  constexpr int PK = SM::PK;
  constexpr int PC = SM::PC;
  __shared__ SM sm;

  const int tid = threadIdx.x;
  const int w = tid >> 6, l = tid & 63, r = l & 15, gq = l >> 4;
  const int H = a.geom.H;
  const int u = blockIdx.x / H;
  const int h = blockIdx.x - u * H;
  if (a.geom.cu != nullptr && u >= *a.geom.n_units) return;  // uniform per workgroup
  const UnitRef U = unit_ref(a.geom, u);
  const int64_t chead = static_cast<int64_t>(u) * H + h;
  st* const oW = static_cast<st*>(a.W);
  st* const oU = static_cast<st*>(a.U);
  st* const oAQ = static_cast<st*>(a.AQ);
  st* const oGQ = static_cast<st*>(a.GQ);
  st* const oLK = static_cast<st*>(a.LK);

  const int c = 16 * w + r;           // my row inside the chunk
  const bool valid = c < U.len;
  const int64_t tok = U.row0 + c;

  // zero T (its above-diagonal blocks are read as zeros by the W/U products)
  for (int i = tid; i < kC * PC; i += 256) sm.Tm[i] = st(0);

  // ---- loads (slot order), masked rows are zero -----------------------------
  float qv[NJ][8], kv[NJ][8], Gt[NJ][8];
  float beta_c = 0.f;
  {
    const int64_t bq = (tok * H + h) * DK;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int ch0 = 32 * j + 4 * gq + 16 * hf;
        f4 x = {0, 0, 0, 0}, y = {0, 0, 0, 0}, z = {0, 0, 0, 0};
        if (valid) {
          x = ld4<DTQ>(a.q, bq + ch0);
          y = ld4<DTQ>(a.k, bq + ch0);
          z = ld4<DTG>(a.g, bq + ch0);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          qv[j][4 * hf + e] = x[e] * a.scale;
          kv[j][4 * hf + e] = y[e];
          Gt[j][4 * hf + e] = z[e] * kLog2e;
        }
      }
    }
    if (valid) beta_c = ld1<DTG>(a.beta, tok * H + h);
  }

  // beta * v  -> BVt (channel-major), done early so v is not kept live
  {
    const int64_t bv = (tok * H + h) * DV;
#pragma unroll
    for (int j = 0; j < NJV; ++j) {
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int ch0 = 32 * j + 4 * gq + 16 * hf;
        f4 x = {0, 0, 0, 0};
        if (valid) x = ld4<DTQ>(a.v, bv + ch0);
#pragma unroll
        for (int e = 0; e < 4; ++e) sm.BVt[(ch0 + e) * PC + c] = st(beta_c * x[e]);
      }
    }
  }

  // ---- tile-local inclusive cumsum (16 rows = 16 lanes of a DPP row) --------
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) Gt[j][e] = row_scan16(Gt[j][e]);

  // k * exp2(Dw - Gt) -> KC (column operand of the off-diagonal score tiles)
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    f8 x;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float dw = row_bcast<15>(Gt[j][e]);
      x[e] = kv[j][e] * fast_exp2(dw - Gt[j][e]);
      if (r == 15) sm.tot[w][32 * j + 8 * gq + e] = Gt[j][e];
    }
    *reinterpret_cast<v8*>(&sm.KC[c * PK + 32 * j + 8 * gq]) = cvt8<EXACT>(x);
  }
  if (gq == 0) sm.beta_s[c] = beta_c;
  __syncthreads();  // #1: tot, KC, BVt, beta_s

  // ---- scores: wave w computes Akk^T / Aqk^T tiles (s, w), s <= w -----------
  f4 accK[4], accQ[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) { accK[s] = f4{0, 0, 0, 0}; accQ[s] = f4{0, 0, 0, 0}; }
  typedef typename Prec<EXACT>::st stt;
  stt lk[NJ][8];  // lambda*k, written to the stage after the scores

#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    float tt[4][8];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int e = 0; e < 8; ++e) tt[t][e] = sm.tot[t][32 * j + 8 * gq + e];

    f8 kr, qr;         // row operands k*exp2(Gt), q*exp2(Gt)
    f8 dk_row, dq_row, dk_col;  // diagonal-tile operands (mid-tile anchor)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float gt = Gt[j][e];
      const float g7 = row_bcast<7>(gt);
      const float R = fast_exp2(gt);
      kr[e] = kv[j][e] * R;
      qr[e] = qv[j][e] * R;
      const float fr = fast_exp2(gt - g7);
      const float fc = fast_exp2(g7 - gt);
      dk_row[e] = kv[j][e] * fr;
      dq_row[e] = qv[j][e] * fr;
      dk_col[e] = kv[j][e] * fc;
    }
    // off-diagonal tiles s < w
#pragma unroll
    for (int s = 0; s < 3; ++s) {
      if (s < w) {
        f8 bk = kr, bqv = qr;
        if (s < w - 1) {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            float m = 0.f;
#pragma unroll
            for (int t = 1; t < 3; ++t)
              if (t > s && t < w) m += tt[t][e];
            const float M = fast_exp2(m);
            bk[e] *= M;
            bqv[e] *= M;
          }
        }
        const v8 A = *reinterpret_cast<const v8*>(&sm.KC[(16 * s + r) * PK + 32 * j + 8 * gq]);
        accK[s] = mma32(accK[s], A, cvt8<EXACT>(bk));
        accQ[s] = mma32(accQ[s], A, cvt8<EXACT>(bqv));
      }
    }
    // diagonal tile s == w
    {
      f4 ak = f4{0, 0, 0, 0}, aq = f4{0, 0, 0, 0};
#pragma unroll
      for (int s = 0; s < 4; ++s) { if (s == w) { ak = accK[s]; aq = accQ[s]; } }
      if constexpr (EXACT) {
        ak = mma32(ak, dk_col, dk_row);
        aq = mma32(aq, dk_col, dq_row);
      } else {
        b8 ah, al, kh, kl, qh, ql;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const __bf16 a0 = static_cast<__bf16>(dk_col[e]);
          ah[e] = a0;
          al[e] = static_cast<__bf16>(dk_col[e] - static_cast<float>(a0));
          const __bf16 k0 = static_cast<__bf16>(dk_row[e]);
          kh[e] = k0;
          kl[e] = static_cast<__bf16>(dk_row[e] - static_cast<float>(k0));
          const __bf16 q0 = static_cast<__bf16>(dq_row[e]);
          qh[e] = q0;
          ql[e] = static_cast<__bf16>(dq_row[e] - static_cast<float>(q0));
        }
        ak = mma32_bf16(ak, ah, kh);
        ak = mma32_bf16(ak, ah, kl);
        ak = mma32_bf16(ak, al, kh);
        aq = mma32_bf16(aq, ah, qh);
        aq = mma32_bf16(aq, ah, ql);
        aq = mma32_bf16(aq, al, qh);
      }
#pragma unroll
      for (int s = 0; s < 4; ++s) { if (s == w) { accK[s] = ak; accQ[s] = aq; } }
    }

    // gamma, lambda for this K step: q*gamma -> GQ (fragment order), the W
    // right-hand side beta*gamma*k -> BWt, lambda*k kept for the stage
    f8 gqv;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float pre = 0.f, post = 0.f;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        if (t < w) pre += tt[t][e];
        if (t > w) post += tt[t][e];
      }
      const float gt = Gt[j][e];
      const float dw = row_bcast<15>(gt);
      const float gam = fast_exp2(pre + gt);
      const float lam = fast_exp2(post + dw - gt);
      gqv[e] = gam * qv[j][e];
      lk[j][e] = stt(lam * kv[j][e]);
      sm.BWt[slot_channel(j, gq, e) * PC + c] = st(beta_c * gam * kv[j][e]);
    }
    *reinterpret_cast<v8*>(oGQ + (chead * (kC / 16) * NJ + (w * NJ + j)) * 512 + l * 8) =
        cvt8<EXACT>(gqv);
    if (w == 0 && r == 0) {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        a.GC[chead * DK + slot_channel(j, gq, e)] =
            fast_exp2(tt[0][e] + tt[1][e] + tt[2][e] + tt[3][e]);
    }
  }

  // masks, L and Aqk fragments
  {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      if (s <= w) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int ii = 4 * gq + i;  // row of the tile = key index i
          if (s == w) {
            if (!(r > ii)) accK[s][i] = 0.f;
            if (!(r >= ii)) accQ[s][i] = 0.f;
          }
        }
        if (s < w) {
          v4 lv;
#pragma unroll
          for (int i = 0; i < 4; ++i) lv[i] = st(beta_c * accK[s][i]);
          *reinterpret_cast<v4*>(&sm.Lm[c * PC + 16 * s + 4 * gq]) = lv;
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) sm.Ld[w][r][4 * gq + i] = beta_c * accK[s][i];
        }
      }
    }
    // Aqk fragments for the state kernel: row tile w, K step jj pairs key tiles (2jj, 2jj+1)
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) {
      f8 x;
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        const int s = 2 * jj + hf;
#pragma unroll
        for (int i = 0; i < 4; ++i) x[4 * hf + i] = (s <= w) ? accQ[s][i] : 0.f;
      }
      *reinterpret_cast<v8*>(oAQ + (chead * (kC / 16) * 2 + (w * 2 + jj)) * 512 + l * 8) =
          cvt8<EXACT>(x);
    }
  }
  __syncthreads();  // #2: Lm, Ld ready; KC free

  // lambda*k -> stage (reuses KC)
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    v8 x;
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = lk[j][e];
    *reinterpret_cast<v8*>(&sm.KC[c * PK + 32 * j + 8 * gq]) = x;
  }

  // diagonal block inverse: lane (any group) computes column r of T_ww
  {
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float acc = 0.f;
#pragma unroll
      for (int m = 0; m < i; ++m) acc += sm.Ld[w][i][m] * x[m];
      x[i] = (i < r) ? 0.f : ((i == r) ? 1.f : -acc);
    }
    if (gq == 0) {
#pragma unroll
      for (int i = 0; i < 16; ++i) sm.Tm[(16 * w + i) * PC + 16 * w + r] = st(x[i]);
    }
  }
  __syncthreads();  // #3: diagonal T blocks, lambda*k stage

  // lambda*k fragments for the state update: (lambda k)^T tile rows = channel
  {
    constexpr int DTW = DK / 64;  // channel tiles per wave
#pragma unroll
    for (int t = 0; t < DTW; ++t) {
      const int dt = w * DTW + t;
      const int d = 16 * dt + r;
      const int jd = d >> 5, wd = d & 31;
      const int sidx = 32 * jd + 8 * ((wd & 15) >> 2) + 4 * (wd >> 4) + (wd & 3);
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        v8 x;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int cc = slot_channel(jj, gq, e);
          x[e] = sm.KC[cc * PK + sidx];
        }
        *reinterpret_cast<v8*>(oLK + (chead * (DK / 16) * 2 + (dt * 2 + jj)) * 512 + l * 8) = x;
      }
    }
  }

  // off-diagonal blocks of T by increasing distance:
  //   T_ws = -T_ww * sum_{j=s}^{w-1} L_wj T_js
#pragma unroll
  for (int dist = 1; dist < 4; ++dist) {
    if (w >= dist) {
      const int s = w - dist;
      f4 X = {0, 0, 0, 0};
      for (int jb = s; jb < w; ++jb) {
        v4 A = *reinterpret_cast<const v4*>(&sm.Lm[(16 * w + r) * PC + 16 * jb + 4 * gq]);
        v4 Bm;
#pragma unroll
        for (int i = 0; i < 4; ++i) Bm[i] = sm.Tm[(16 * jb + 4 * gq + i) * PC + 16 * s + r];
        X = mma16(X, A, Bm);
      }
      v4 A2 = *reinterpret_cast<const v4*>(&sm.Tm[(16 * w + r) * PC + 16 * w + 4 * gq]);
      f4 Y = mma16(f4{0, 0, 0, 0}, A2, cvt4<EXACT>(X));
#pragma unroll
      for (int i = 0; i < 4; ++i) sm.Tm[(16 * w + 4 * gq + i) * PC + 16 * s + r] = st(-Y[i]);
    }
    __syncthreads();  // #4..#6
  }

  // ---- W^T tiles and U tiles for row tile w ---------------------------------
  const int nk = (w < 2) ? 1 : 2;
#pragma unroll
  for (int dt = 0; dt < DK / 16; ++dt) {
    f4 acc = {0, 0, 0, 0};
    for (int jc = 0; jc < nk; ++jc) {
      const v8 A = *reinterpret_cast<const v8*>(&sm.BWt[(16 * dt + r) * PC + 32 * jc + 8 * gq]);
      const v8 B = *reinterpret_cast<const v8*>(&sm.Tm[(16 * w + r) * PC + 32 * jc + 8 * gq]);
      acc = mma32(acc, A, B);
    }
    *reinterpret_cast<v4*>(oW + (chead * (kC / 16) * NJ + (w * NJ + (dt >> 1))) * 512 + l * 8 +
                           (dt & 1) * 4) = cvt4<EXACT>(acc);
  }
#pragma unroll
  for (int et = 0; et < DV / 16; ++et) {
    f4 acc = {0, 0, 0, 0};
    for (int jc = 0; jc < nk; ++jc) {
      const v8 A = *reinterpret_cast<const v8*>(&sm.Tm[(16 * w + r) * PC + 32 * jc + 8 * gq]);
      const v8 B = *reinterpret_cast<const v8*>(&sm.BVt[(16 * et + r) * PC + 32 * jc + 8 * gq]);
      acc = mma32(acc, A, B);
    }
    *reinterpret_cast<v4*>(oU + (chead * (kC / 16) * (DV / 16) + (w * (DV / 16) + et)) * 256 +
                           l * 4) = cvt4<EXACT>(acc);
  }
}

// ----------------------------------------------------------------------------
// State kernel: serial over the chunks of one chain, 32 value columns per WG
// ----------------------------------------------------------------------------
template <int DK, int DV, bool EXACT, int OUT_DT>
__global__ __launch_bounds__(256, 1)
void kda_state_kernel(StateArgs a) {
  typedef typename Prec<EXACT>::st st;
  typedef typename Prec<EXACT>::v8 v8;
  typedef typename Prec<EXACT>::v4 v4;
  constexpr int NJ = DK / 32;
  constexpr int SPLITS = DV / 32;
  constexpr int DTW = DK / 64;          // state channel tiles per wave
  constexpr int PK = DK + 8;
  constexpr int PC = kC + 8;
  __shared__ st St[32 * PK];            // S^T slice: [value col][channel]
  __shared__ st Vt[32 * PC];            // v~^T: [value col][row]

  const int tid = threadIdx.x;
  const int w = tid >> 6, l = tid & 63, r = l & 15, gq = l >> 4;
  const Geom& G = a.geom;
  const int H = G.H;

  // XCD-aware mapping: the SPLITS workgroups of one chain share an XCD (and L2)
  const st* const iW = static_cast<const st*>(a.W);
  const st* const iU = static_cast<const st*>(a.U);
  const st* const iAQ = static_cast<const st*>(a.AQ);
  const st* const iGQ = static_cast<const st*>(a.GQ);
  const st* const iLK = static_cast<const st*>(a.LK);
  const int x = blockIdx.x;
  const int xcd = x & 7;
  const int kk = x >> 3;
  const int slot = kk / SPLITS;
  const int split = kk - slot * SPLITS;
  const int chain = slot * 8 + xcd;
  if (chain >= G.N * H) return;
  const int seq_rank = chain / H;
  const int h = chain - seq_rank * H;
  const int seq = (G.order != nullptr) ? G.order[seq_rank] : seq_rank;

  int u0, nchunks;
  int64_t tok0;
  int seq_len;
  if (G.cu == nullptr) {
    u0 = seq * G.NT;
    nchunks = G.NT;
    tok0 = static_cast<int64_t>(seq) * G.T;
    seq_len = G.T;
  } else {
    u0 = G.chunk_off[seq];
    nchunks = G.chunk_off[seq + 1] - u0;
    tok0 = G.cu_clamped[seq];
    seq_len = G.cu_clamped[seq + 1] - G.cu_clamped[seq];
  }

  // state accumulators: tiles (dt = w*DTW + t, et), rows 4*gq+i, column r
  f4 S[DTW][2];
  const int64_t sbase = (static_cast<int64_t>(seq) * H + h) * DK * DV;
#pragma unroll
  for (int t = 0; t < DTW; ++t)
#pragma unroll
    for (int et = 0; et < 2; ++et)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = 16 * (w * DTW + t) + 4 * gq + i;
        const int e = 32 * split + 16 * et + r;
        S[t][et][i] = (a.h0 != nullptr) ? a.h0[sbase + static_cast<int64_t>(d) * DV + e] : 0.f;
      }

  for (int n = 0; n < nchunks; ++n) {
    const int64_t chead = static_cast<int64_t>(u0 + n) * H + h;
    const int64_t row0 = tok0 + static_cast<int64_t>(n) * kC;
    const int len = min(kC, static_cast<int>(seq_len - static_cast<int64_t>(n) * kC));

    // operands of this chunk (fragment order, written by the intra kernel)
    v8 Wf[NJ], Qf[NJ], Af[2], Lf[DTW][2];
    v4 Uf[2];
    f4 gc[DTW];
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      Wf[j] = *reinterpret_cast<const v8*>(iW + (chead * (kC / 16) * NJ + (w * NJ + j)) * 512 + l * 8);
      Qf[j] = *reinterpret_cast<const v8*>(iGQ + (chead * (kC / 16) * NJ + (w * NJ + j)) * 512 + l * 8);
    }
#pragma unroll
    for (int jj = 0; jj < 2; ++jj)
      Af[jj] = *reinterpret_cast<const v8*>(iAQ + (chead * (kC / 16) * 2 + (w * 2 + jj)) * 512 + l * 8);
#pragma unroll
    for (int et = 0; et < 2; ++et)
      Uf[et] = *reinterpret_cast<const v4*>(
          iU + (chead * (kC / 16) * (DV / 16) + (w * (DV / 16) + 2 * split + et)) * 256 + l * 4);
#pragma unroll
    for (int t = 0; t < DTW; ++t) {
      const int dt = w * DTW + t;
#pragma unroll
      for (int jj = 0; jj < 2; ++jj)
        Lf[t][jj] = *reinterpret_cast<const v8*>(iLK + (chead * (DK / 16) * 2 + (dt * 2 + jj)) * 512 + l * 8);
      gc[t] = *reinterpret_cast<const f4*>(a.GC + chead * DK + 16 * dt + 4 * gq);
    }

    // 1. S^T slice -> LDS (operand precision)
#pragma unroll
    for (int t = 0; t < DTW; ++t)
#pragma unroll
      for (int et = 0; et < 2; ++et)
        *reinterpret_cast<v4*>(&St[(16 * et + r) * PK + 16 * (w * DTW + t) + 4 * gq]) = cvt4<EXACT>(S[t][et]);
    __syncthreads();

    // 2. P = W S, O = (gamma q) S, v~ = U - P
    f4 O[2];
#pragma unroll
    for (int et = 0; et < 2; ++et) {
      f4 P = {0, 0, 0, 0};
      O[et] = f4{0, 0, 0, 0};
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        v8 Sf;
        const st* row = &St[(16 * et + r) * PK + 32 * j + 4 * gq];
        const v4 s0 = *reinterpret_cast<const v4*>(row);
        const v4 s1 = *reinterpret_cast<const v4*>(row + 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) { Sf[i] = s0[i]; Sf[4 + i] = s1[i]; }
        P = mma32(P, Wf[j], Sf);
        O[et] = mma32(O[et], Qf[j], Sf);
      }
      f4 vt;
#pragma unroll
      for (int i = 0; i < 4; ++i) vt[i] = static_cast<float>(Uf[et][i]) - P[i];
      *reinterpret_cast<v4*>(&Vt[(16 * et + r) * PC + 16 * w + 4 * gq]) = cvt4<EXACT>(vt);
    }
    __syncthreads();

    // 3. O += Aqk v~ ; 4. S <- gamma_C S + (lambda k)^T v~
    const int nk2 = (w < 2) ? 1 : 2;
#pragma unroll
    for (int et = 0; et < 2; ++et) {
      v8 Vf[2];
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const st* row = &Vt[(16 * et + r) * PC + 32 * jj + 4 * gq];
        const v4 s0 = *reinterpret_cast<const v4*>(row);
        const v4 s1 = *reinterpret_cast<const v4*>(row + 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) { Vf[jj][i] = s0[i]; Vf[jj][4 + i] = s1[i]; }
      }
      for (int jj = 0; jj < nk2; ++jj) O[et] = mma32(O[et], Af[jj], Vf[jj]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int cr = 16 * w + 4 * gq + i;
        if (cr < len) {
          const int64_t oi = ((row0 + cr) * H + h) * DV + 32 * split + 16 * et + r;
          if constexpr (OUT_DT == 0) static_cast<float*>(a.o)[oi] = O[et][i];
          else static_cast<u16*>(a.o)[oi] = f32_to_bf16_bits(O[et][i]);
        }
      }
#pragma unroll
      for (int t = 0; t < DTW; ++t) {
        f4 s = S[t][et];
#pragma unroll
        for (int i = 0; i < 4; ++i) s[i] *= gc[t][i];
        s = mma32(s, Lf[t][0], Vf[0]);
        s = mma32(s, Lf[t][1], Vf[1]);
        S[t][et] = s;
      }
    }
    // (the next iteration's first barrier orders Vt/St reuse)
  }

  if (a.ht != nullptr) {
#pragma unroll
    for (int t = 0; t < DTW; ++t)
#pragma unroll
      for (int et = 0; et < 2; ++et)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int d = 16 * (w * DTW + t) + 4 * gq + i;
          const int e = 32 * split + 16 * et + r;
          a.ht[sbase + static_cast<int64_t>(d) * DV + e] = S[t][et][i];
        }
  }
}

// ----------------------------------------------------------------------------
// varlen preparation: clamp cu_seqlens, chunk offsets, longest-first order
// ----------------------------------------------------------------------------
__global__ __launch_bounds__(1024)
void kda_varlen_prep_kernel(const int32_t* cu, int N, int T, int32_t* cu_clamped,
                            int32_t* chunk_off, int32_t* n_units, int32_t* order,
                            int32_t* flags) {
  __shared__ int32_t scan[1024];
  __shared__ int32_t carry;
  __shared__ int32_t bad;
  __shared__ int64_t keys[2048];
  const int tid = threadIdx.x;
  if (tid == 0) { carry = 0; bad = 0; }
  __syncthreads();
  // clamp: 0 <= cu[i] <= T and non-decreasing; flag any repair
  for (int base = 0; base <= N; base += 1024) {
    const int i = base + tid;
    int v = 0;
    if (i <= N) {
      v = cu[i];
      int lo = (i == 0) ? 0 : cu[i - 1];
      if (i == 0 && v != 0) atomicOr(&bad, 1);
      if (i == N && v != T) atomicOr(&bad, 2);
      if (v < lo) { atomicOr(&bad, 4); }
      if (v < 0 || v > T) atomicOr(&bad, 8);
    }
    (void)v;
  }
  __syncthreads();
  // serial-safe clamp in one thread group pass (running max)
  for (int base = 0; base <= N; base += 1024) {
    const int i = base + tid;
    int v = 0;
    if (i <= N) v = min(max(cu[i], 0), T);
    if (i == 0) v = 0;
    scan[tid] = v;
    __syncthreads();
    // inclusive running max (Hillis-Steele)
    for (int off = 1; off < 1024; off <<= 1) {
      int t = (tid >= off) ? scan[tid - off] : 0;
      __syncthreads();
      scan[tid] = max(scan[tid], t);
      __syncthreads();
    }
    const int m = max(scan[tid], carry);
    if (i <= N) cu_clamped[i] = m;
    __syncthreads();
    if (tid == 1023) carry = m;
    __syncthreads();
  }
  if (tid == 0) carry = 0;
  __syncthreads();
  // chunk offsets: exclusive scan of ceil(len/64)
  for (int base = 0; base < N; base += 1024) {
    const int i = base + tid;
    int cnt = 0;
    if (i < N) cnt = (cu_clamped[i + 1] - cu_clamped[i] + kC - 1) / kC;
    scan[tid] = cnt;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {
      int t = (tid >= off) ? scan[tid - off] : 0;
      __syncthreads();
      scan[tid] += t;
      __syncthreads();
    }
    if (i < N) chunk_off[i] = carry + scan[tid] - cnt;
    __syncthreads();
    if (tid == 1023) carry += scan[1023];
    __syncthreads();
  }
  if (tid == 0) { chunk_off[N] = carry; *n_units = carry; flags[0] = bad; }
  // longest-first order (bitonic sort of (-len, idx)); identity for large N
  if (N <= 2048) {
    for (int i = tid; i < 2048; i += 1024) {
      if (i < N) {
        const int64_t len = cu_clamped[i + 1] - cu_clamped[i];
        keys[i] = ((int64_t)(0x7FFFFFFF - len) << 32) | (uint32_t)i;
      } else {
        keys[i] = INT64_MAX;
      }
    }
    __syncthreads();
    for (int k = 2; k <= 2048; k <<= 1) {
      for (int j = k >> 1; j > 0; j >>= 1) {
        for (int i = tid; i < 2048; i += 1024) {
          const int ixj = i ^ j;
          if (ixj > i) {
            const bool up = ((i & k) == 0);
            const int64_t a0 = keys[i], a1 = keys[ixj];
            if ((a0 > a1) == up) { keys[i] = a1; keys[ixj] = a0; }
          }
        }
        __syncthreads();
      }
    }
    for (int i = tid; i < N; i += 1024) order[i] = (int32_t)(keys[i] & 0xFFFFFFFF);
  } else {
    for (int i = tid; i < N; i += 1024) order[i] = i;
  }
}

// ----------------------------------------------------------------------------
// host-side launchers
// ----------------------------------------------------------------------------
template <int DK, int DV, int DTQ, int DTG, bool EXACT>
static hipError_t launch_intra_t(const IntraArgs& a, int grid, hipStream_t s) {
  hipLaunchKernelGGL((kda_intra_kernel<DK, DV, DTQ, DTG, EXACT>), dim3(grid), dim3(256), 0, s, a);
  return hipGetLastError();
}

template <int DK, int DV, bool EXACT, int OUT>
static hipError_t launch_state_t(const StateArgs& a, int grid, hipStream_t s) {
  hipLaunchKernelGGL((kda_state_kernel<DK, DV, EXACT, OUT>), dim3(grid), dim3(256), 0, s, a);
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

hipError_t launch_varlen_prep(const int32_t* cu, int N, int T, int32_t* cu_clamped,
                              int32_t* chunk_off, int32_t* n_units, int32_t* order,
                              int32_t* flags, hipStream_t s) {
  hipLaunchKernelGGL(kda_varlen_prep_kernel, dim3(1), dim3(1024), 0, s, cu, N, T, cu_clamped,
                     chunk_off, n_units, order, flags);
  return hipGetLastError();
}

}  // namespace kda
