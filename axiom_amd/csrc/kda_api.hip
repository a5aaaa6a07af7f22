// C ABI of the KDA hot path: argument validation, workspace layout, dispatch.
#include "kda_mi355x.h"

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <initializer_list>
#include <numeric>

#include "kda_common.h"
#include "kda_internal.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(KDA_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

constexpr int kC = 64;
constexpr size_t kAlign = 256;

size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

struct WsLayout {
  size_t W, U, AQ, GQ, LK, GC;
  size_t cu_clamped, chunk_off, n_units, order, flags;
  size_t state;          // carried state between segments (segmented calls)
  size_t pos_off, seg_pos;  // position-major unit tables (segmented varlen calls)
  int vsegs;             // varlen: launches (1 = every unit at once)
  int KU;                // varlen, segmented: units per launch
  size_t status;         // int32 status word of the call (kda::kStatusNonFinite)
  size_t total;
  int64_t units_bound;   // workspace chunk units (per segment when segmented)
  int segments;          // dense: launches along T (1 = whole sequence at once)
  int seg_chunks;        // dense: chunks per segment
  int bufs;              // 2: segments alternate between two sets of intra results
  size_t sz_W, sz_U, sz_AQ, sz_GQ, sz_LK, sz_GC;  // bytes of one set
};

bool is_exact(int in_dtype) { return in_dtype == KDA_DTYPE_F32; }

// Bytes of intra-chunk results per chunk-head (W, gamma*q, lambda*k, U, Aqk,
// gamma_C), before alignment.
size_t bytes_per_chunk_head(int dk, int dv, size_t es) {
  return static_cast<size_t>(kC) * (3 * dk + dv + kC) * es + static_cast<size_t>(dk) * 4;
}

// Dense calls run the sequence in segments of chunks (intra then state per
// segment, the state carried between them) so that one segment's
// intra-chunk results stay within this budget: on MI355X they are then read
// back by the state kernel from the 256 MB last-level cache rather than
// HBM, and the next segment overwrites them there.  Config 1 (B4 T4096 H16
// d128, 304 MB of results) runs as 2 segments of 32 chunks: 206 us against
// 212 us as 3 (24 + 24 + 16) and 241 us unsegmented, measured once the
// intra kernel's input copies were non-temporal (they no longer compete
// with the results for the cache; before that 3 segments were best: 282 us
// against 287 for 2 and 305 unsegmented).
constexpr double kSegmentBudgetBytes = 160.0 * 1048576.0;
// Intra workgroups resident at once (two on each of the MI355X's 256 CUs).
// A segment's chunk count is rounded up so its B * H * chunks workgroups fill
// whole rounds of them (measured when config 1 ran 3 segments: 24 + 24 + 16
// chunks, 227.6 us, against 22 + 22 + 20, 232.9 us, whose last round per
// segment ran a quarter empty).
constexpr int kIntraSlots = 512;

// Overlapped segments (the state scan of segment s in the same launch as the
// intra-chunk work of segment s+1) when the state kernel's grid leaves most
// of the chip free: at most this many 32-column state workgroups (each holds a
// CU for the whole segment; 24 chains at dv = 128).  Both segments' intra
// results then live at once, next to the inputs the intra work streams, so a
// segment's budget is smaller.  Config 2 (B1 T65536 H16), with the intra
// kernel's input copies non-temporal: 1 134 us overlapped at 96 MiB (48:
// 1 166, 56: 1 161, 64: 1 148, 80: 1 143, 112: 1 136, 128: 1 141); before
// those copies were non-temporal the inputs competed for the 256 MB
// memory-side cache and 48 MiB was best (1 239 us; 100 MiB: 1 915 us, the
// serial scan waiting on HBM; sequential 100 MiB segments: 1 530 us).  At
// 128 state workgroups (32 chains) overlapping gained nothing (1 085 against
// 1 085 us), at 96 (24 chains) 1 855 -> 1 770 us.
constexpr int64_t kOverlapMaxStateWgs = 96;

// A varlen call runs every chunk-head at once when its workspace allows
// (kda_chunk_fwd_workspace: the fastest schedule), else in segments of KU
// units of a position-major numbering (every sequence's chunk p before any
// sequence's chunk p + 1, sequences longest-first), the largest KU whose
// layout fits the caller's workspace; each chain's state crosses the
// segment boundaries in ht (or a workspace copy), as in the segmented dense
// calls.  The least workspace accepted (kda_chunk_fwd_workspace_min) holds
// this budget of intra-chunk results per segment.  Segmenting trades time
// for memory: config 3 (64 sequences, T = 309 178) 3 902 us in one launch
// pair (5.8 GB of workspace), 4 059 / 4 156 / 4 163 / 4 657 us in segments
// of 1 280 / 640 / 320 / 160 MiB of results (each chain restarts its scan
// at every boundary and the last positions are walked by few chains).  Needs
// the longest-first order (at most 2 048 sequences: the prep kernel's sort).
constexpr double kVarlenSegmentBudgetBytes = 160.0 * 1048576.0;
constexpr int kVarlenSegmentMaxSeqs = 2048;
constexpr double kOverlapSegmentBudgetBytes = 96.0 * 1048576.0;

int64_t col_state_grid(int64_t chains, int dv) { return ((chains + 7) / 8) * 8 * (dv / 32); }

bool overlap_eligible(int B, int H, int dv, int in_dtype) {
  return !is_exact(in_dtype) && col_state_grid(static_cast<int64_t>(B) * H, dv) <= kOverlapMaxStateWgs;
}

int dense_segments(int B, int T, int H, int dk, int dv, int in_dtype) {
  const int NT = (T + kC - 1) / kC;
  if (NT <= 1) return 1;
  const size_t es = is_exact(in_dtype) ? 4 : 2;
  const double total = static_cast<double>(B) * NT * H * bytes_per_chunk_head(dk, dv, es);
  const double budget = overlap_eligible(B, H, dv, in_dtype) ? kOverlapSegmentBudgetBytes : kSegmentBudgetBytes;
  int s = static_cast<int>(std::ceil(total / budget));
  // An overlapped call of one segment's worth still runs as two: the second
  // half's intra work then hides under the first half's scan (B1 T4096 H16:
  // 97 -> 89 us; four segments: 98 us).
  if (overlap_eligible(B, H, dv, in_dtype) && s < 2 && NT >= 32) s = 2;
  return s < 1 ? 1 : (s > NT ? NT : s);
}

// upper bound on a varlen call's chunk units: sum ceil(len_i / C) <= (T + (C-1) N) / C
int64_t varlen_units(int T, int32_t n_seqs) { return (static_cast<int64_t>(T) + 63LL * n_seqs) / kC; }

// n_seqs <= 0: dense.  Varlen: ku = 0 runs every unit in one launch pair,
// ku > 0 (below the unit bound; at most 2 048 sequences) runs segments of ku
// units.
WsLayout ws_layout(int B, int T, int H, int dk, int dv, int32_t n_seqs, int in_dtype, int64_t ku = 0) {
  WsLayout L{};
  const size_t es = is_exact(in_dtype) ? 4 : 2;
  int64_t units;
  L.segments = 1;
  L.vsegs = 1;
  L.KU = 0;
  L.seg_chunks = (T + kC - 1) / kC;
  if (n_seqs > 0) {
    units = varlen_units(T, n_seqs);
    if (ku > 0 && ku < units && n_seqs <= kVarlenSegmentMaxSeqs) {
      L.KU = static_cast<int>(ku);
      L.vsegs = static_cast<int>((units + ku - 1) / ku);
      units = ku;
    }
  } else {
    const int NT = L.seg_chunks;
    L.segments = dense_segments(B, T, H, dk, dv, in_dtype);
    L.seg_chunks = (L.seg_chunks + L.segments - 1) / L.segments;
    if (L.segments > 1 && !overlap_eligible(B, H, dv, in_dtype)) {
      const int64_t bh = static_cast<int64_t>(B) * H;
      const int m = static_cast<int>(kIntraSlots / std::gcd<int64_t>(kIntraSlots, bh));
      const int up = (L.seg_chunks + m - 1) / m * m;
      if (up < NT) L.seg_chunks = up;
    }
    L.segments = (L.seg_chunks > 0) ? (NT + L.seg_chunks - 1) / L.seg_chunks : 1;
    units = static_cast<int64_t>(B) * L.seg_chunks;
  }
  L.units_bound = units;
  L.bufs = (n_seqs <= 0 && L.segments > 1 && overlap_eligible(B, H, dv, in_dtype)) ? 2 : 1;
  const int64_t ch = units * H;
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t at = off; off = align_up(off + bytes); return at; };
  L.sz_W = L.sz_GQ = L.sz_LK = align_up(static_cast<size_t>(ch) * kC * dk * es);
  L.sz_U = align_up(static_cast<size_t>(ch) * kC * dv * es);
  L.sz_AQ = align_up(static_cast<size_t>(ch) * kC * kC * es);
  L.sz_GC = align_up(static_cast<size_t>(ch) * dk * 4);
  L.W = take(L.sz_W * L.bufs);
  L.GQ = take(L.sz_GQ * L.bufs);
  L.LK = take(L.sz_LK * L.bufs);
  L.U = take(L.sz_U * L.bufs);
  L.AQ = take(L.sz_AQ * L.bufs);
  L.GC = take(L.sz_GC * L.bufs);
  if (n_seqs > 0) {
    L.cu_clamped = take(static_cast<size_t>(n_seqs + 1) * 4);
    L.chunk_off = take(static_cast<size_t>(n_seqs + 1) * 4);
    L.n_units = take(4);
    L.order = take(static_cast<size_t>(n_seqs) * 4);
    L.flags = take(4);
    if (L.vsegs > 1) {
      L.pos_off = take((static_cast<size_t>(T + kC - 1) / kC + 2) * 4);
      L.seg_pos = take(static_cast<size_t>(L.vsegs + 1) * 2 * 4);
    }
  }
  if (L.segments > 1 || L.vsegs > 1)
    L.state = take(static_cast<size_t>(n_seqs > 0 ? n_seqs : B) * H * dk * dv * 4);
  L.status = take(4);
  L.total = off;
  return L;
}

// Units per segment of a varlen call's smallest workspace (the budget's
// worth of intra-chunk results), or 0 when the call runs unsegmented anyway.
int64_t varlen_min_ku(int T, int H, int dk, int dv, int32_t n_seqs, int in_dtype) {
  const int64_t units = varlen_units(T, n_seqs);
  const double per_unit = static_cast<double>(H) * bytes_per_chunk_head(dk, dv, is_exact(in_dtype) ? 4 : 2);
  if (n_seqs > kVarlenSegmentMaxSeqs || static_cast<double>(units) * per_unit <= kVarlenSegmentBudgetBytes) return 0;
  return std::max<int64_t>(1, static_cast<int64_t>(kVarlenSegmentBudgetBytes / per_unit));
}

// The layout a call with ws_bytes of workspace runs: the fastest one when it
// fits, else (varlen) the segments of the most units that fit.  ok = false:
// not even the smallest layout fits.
WsLayout ws_layout_for(int B, int T, int H, int dk, int dv, int32_t n_seqs, int in_dtype, size_t ws_bytes,
                       bool* ok) {
  const WsLayout full = ws_layout(B, T, H, dk, dv, n_seqs, in_dtype);
  *ok = true;
  if (ws_bytes >= full.total || n_seqs <= 0) {
    *ok = ws_bytes >= full.total;
    return full;
  }
  const int64_t kmin = varlen_min_ku(T, H, dk, dv, n_seqs, in_dtype);
  if (kmin == 0 || ws_layout(B, T, H, dk, dv, n_seqs, in_dtype, kmin).total > ws_bytes) {
    *ok = false;
    return full;
  }
  // largest ku in [kmin, units) whose layout fits (the size grows with ku)
  int64_t lo = kmin, hi = varlen_units(T, n_seqs) - 1;
  while (lo < hi) {
    const int64_t mid = lo + (hi - lo + 1) / 2;
    if (ws_layout(B, T, H, dk, dv, n_seqs, in_dtype, mid).total <= ws_bytes) lo = mid; else hi = mid - 1;
  }
  return ws_layout(B, T, H, dk, dv, n_seqs, in_dtype, lo);
}

bool dim_ok(int d) { return d == 64 || d == 128; }

// The kernels move rows, fragments and state slices 16 bytes (bf16 v in
// decode: 8 bytes) per lane access, so those pointers must be aligned to
// that; a null pointer is left to the null checks.
bool misaligned(const void* p, uintptr_t bytes) { return (reinterpret_cast<uintptr_t>(p) & (bytes - 1)) != 0; }

// Every pointer of `ps` aligned to `bytes` (null pointers pass), else a
// KDA_ERR_INVALID_ARGUMENT naming `what`.
int require_aligned(uintptr_t bytes, const char* what, std::initializer_list<const void*> ps) {
  for (const void* p : ps)
    if (misaligned(p, bytes)) return fail(KDA_ERR_INVALID_ARGUMENT, "%s must be %d-byte aligned", what, static_cast<int>(bytes));
  return KDA_OK;
}

// bytes of four elements of a kda_dtype_t that is F32 or BF16
uintptr_t four_elems(int dtype) { return dtype == KDA_DTYPE_F32 ? 16 : 8; }

int check_dims(int H, int dk, int dv) {
  if (H < 1) return fail(KDA_ERR_INVALID_ARGUMENT, "H=%d must be >= 1", H);
  if (dk < 1 || dv < 1) return fail(KDA_ERR_INVALID_ARGUMENT, "dk=%d, dv=%d must be >= 1", dk, dv);
  if (!dim_ok(dk) || dk != dv)
    return fail(KDA_ERR_UNSUPPORTED, "head dims dk=%d, dv=%d: this build runs dk == dv in {64, 128}", dk, dv);
  return KDA_OK;
}

template <typename T>
T* at(void* base, size_t off) { return reinterpret_cast<T*>(static_cast<char*>(base) + off); }

// The layer's short conv fused into the intra kernel (q, k, v are then the
// raw projections): taps and first-chunk history per tensor, K taps.
struct FusedPrologue {
  const float* cw[3];
  const float* cb[3];
  int K;
};

int chunk_fwd_impl(hipStream_t stream, const void* q, const void* k, const void* v,
                   const void* g, const void* beta, const float* h0,
                   const int32_t* cu_seqlens, int32_t n_seqs, void* o, float* ht,
                   int B, int T, int H, int dk, int dv, int chunk, float scale,
                   int in_dtype, int out_dtype, void* ws, size_t ws_bytes,
                   const FusedPrologue* pro = nullptr, bool gates_alpha = false) {
  if (!q || !k || !v || !g || !beta) return fail(KDA_ERR_INVALID_ARGUMENT, "null input pointer");
  if (!o && T > 0) return fail(KDA_ERR_INVALID_ARGUMENT, "null output pointer o");
  if (B < 1) return fail(KDA_ERR_INVALID_ARGUMENT, "B=%d must be >= 1", B);
  if (T < 0) return fail(KDA_ERR_INVALID_ARGUMENT, "T=%d must be >= 0", T);
  if (int rc = check_dims(H, dk, dv)) return rc;
  if (chunk != kC) return fail(KDA_ERR_UNSUPPORTED, "chunk=%d: this build runs chunk == 64", chunk);
  if (in_dtype < KDA_DTYPE_F32 || in_dtype > KDA_DTYPE_BF16_F32GATES)
    return fail(KDA_ERR_INVALID_ARGUMENT, "in_dtype=%d is not a kda_dtype_t", in_dtype);
  if (out_dtype != KDA_DTYPE_F32 && out_dtype != KDA_DTYPE_BF16)
    return fail(KDA_ERR_INVALID_ARGUMENT, "out_dtype=%d: o is emitted as F32 or BF16", out_dtype);
  if (!std::isfinite(scale)) return fail(KDA_ERR_INVALID_ARGUMENT, "scale must be finite");
  const bool varlen = cu_seqlens != nullptr;
  if (varlen) {
    if (B != 1) return fail(KDA_ERR_INVALID_ARGUMENT, "cu_seqlens requires B == 1 (got B=%d)", B);
    if (n_seqs < 1) return fail(KDA_ERR_INVALID_ARGUMENT, "n_seqs=%d must be >= 1 with cu_seqlens", n_seqs);
  }
  const int64_t elems = static_cast<int64_t>(B) * T * H * (dk > dv ? dk : dv);
  if (elems >= (1LL << 40)) return fail(KDA_ERR_INVALID_ARGUMENT, "problem too large");
  if (misaligned(q, 16) || misaligned(k, 16) || misaligned(v, 16) || misaligned(g, 16) || misaligned(o, 16) ||
      misaligned(ws, 16) || (gates_alpha && misaligned(beta, 16)))
    return fail(KDA_ERR_INVALID_ARGUMENT, "q, k, v, g%s, o and the workspace must be 16-byte aligned",
                gates_alpha ? ", beta32" : "");
  bool fits = false;
  const WsLayout L = ws_layout_for(B, T, H, dk, dv, varlen ? n_seqs : 0, in_dtype, ws ? ws_bytes : 0, &fits);
  if (L.units_bound * H > 0x7FFFFFFFLL) return fail(KDA_ERR_INVALID_ARGUMENT, "too many chunk-heads");
  if (ws == nullptr || !fits) {
    const int64_t kmin = varlen ? varlen_min_ku(T, H, dk, dv, n_seqs, in_dtype) : 0;
    const size_t least = kmin > 0 ? ws_layout(B, T, H, dk, dv, n_seqs, in_dtype, kmin).total : L.total;
    return fail(KDA_ERR_WORKSPACE, "workspace of %zu bytes is too small (need %zu)", ws ? ws_bytes : 0, least);
  }

  const bool exact = is_exact(in_dtype);
  int dtq, dtg;
  switch (in_dtype) {
    case KDA_DTYPE_F32: dtq = 0; dtg = 0; break;
    case KDA_DTYPE_BF16: dtq = 1; dtg = 1; break;
    case KDA_DTYPE_F16: dtq = 2; dtg = 2; break;
    default: dtq = 1; dtg = 0; break;
  }

  kda::Geom G{};
  G.B = B; G.T = T; G.H = H;
  G.NT = (T + kC - 1) / kC;
  G.n0 = 0;
  G.NTS = G.NT;
  G.N = varlen ? n_seqs : B;
  if (varlen) {
    G.cu = cu_seqlens;
    G.cu_clamped = at<int32_t>(ws, L.cu_clamped);
    G.chunk_off = at<int32_t>(ws, L.chunk_off);
    G.n_units = at<int32_t>(ws, L.n_units);
    G.order = at<int32_t>(ws, L.order);
    if (L.vsegs > 1) {
      G.pos_off = at<int32_t>(ws, L.pos_off);
      G.seg_pos = at<int32_t>(ws, L.seg_pos);
      G.KU = L.KU;
    }
    hipError_t e = kda::launch_varlen_prep(cu_seqlens, n_seqs, T, at<int32_t>(ws, L.cu_clamped),
                                           at<int32_t>(ws, L.chunk_off), at<int32_t>(ws, L.n_units),
                                           at<int32_t>(ws, L.order), at<int32_t>(ws, L.flags),
                                           L.vsegs > 1 ? at<int32_t>(ws, L.pos_off) : nullptr,
                                           L.vsegs > 1 ? at<int32_t>(ws, L.seg_pos) : nullptr, L.KU, L.vsegs,
                                           stream);
    if (e != hipSuccess) return hip_fail(e, "varlen prep launch");
  }

  kda::IntraArgs ia{};
  ia.geom = G;
  ia.q = q; ia.k = k; ia.v = v; ia.g = g; ia.beta = beta;
  ia.scale = scale;
  ia.gates_alpha = gates_alpha ? 1 : 0;
  ia.W = at<void>(ws, L.W);
  ia.U = at<void>(ws, L.U);
  ia.AQ = at<void>(ws, L.AQ);
  ia.GQ = at<void>(ws, L.GQ);
  ia.LK = at<void>(ws, L.LK);
  ia.GC = at<float>(ws, L.GC);
  if (pro != nullptr) {
    for (int t = 0; t < 3; ++t) { ia.cw[t] = pro->cw[t]; ia.cb[t] = pro->cb[t]; }
    ia.K = pro->K;
  }

  // the call's status word: zeroed by the first intra launch, set by the
  // 16-bit state kernels on a non-finite o or final state value
  int* const status = at<int>(ws, L.status);
  ia.status_clear = status;

  kda::StateArgs sa{};
  sa.geom = G;
  sa.W = ia.W; sa.U = ia.U; sa.AQ = ia.AQ; sa.GQ = ia.GQ; sa.LK = ia.LK; sa.GC = ia.GC;
  sa.o = o;
  sa.status = exact ? nullptr : status;
  const int64_t chains = static_cast<int64_t>(G.N) * H;
  const int64_t state_grid = col_state_grid(chains, dv);
  if (state_grid > 0x7FFFFFFFLL) return fail(KDA_ERR_INVALID_ARGUMENT, "too many chains");

  // Segments along T (dense only): the state leaves one segment in `carry`
  // and enters the next from it (each state workgroup reads its slice before
  // writing it, so the same buffer serves as both).
  float* carry = (L.segments > 1) ? (ht != nullptr ? ht : at<float>(ws, L.state)) : ht;
  const int out_dt = out_dtype == KDA_DTYPE_BF16 ? 1 : 0;
  if (!varlen && pro == nullptr && L.bufs == 2) {
    // Overlapped segments: intra(0); then per launch the state scan of
    // segment s (results set s % 2) and the intra work of segment s+1 (set
    // (s+1) % 2); then the state scan of the last segment.
    auto set_bufs = [&](int b) {
      ia.W = at<char>(ws, L.W) + b * L.sz_W;
      ia.GQ = at<char>(ws, L.GQ) + b * L.sz_GQ;
      ia.LK = at<char>(ws, L.LK) + b * L.sz_LK;
      ia.U = at<char>(ws, L.U) + b * L.sz_U;
      ia.AQ = at<char>(ws, L.AQ) + b * L.sz_AQ;
      ia.GC = reinterpret_cast<float*>(at<char>(ws, L.GC) + b * L.sz_GC);
    };
    auto seg_geom = [&](int sgi) {
      kda::Geom g2 = G;
      g2.n0 = sgi * L.seg_chunks;
      g2.NTS = std::min(L.seg_chunks, G.NT - g2.n0);
      return g2;
    };
    set_bufs(0);
    ia.geom = seg_geom(0);
    hipError_t e = kda::launch_intra(ia, dk, dtq, dtg, static_cast<int>(static_cast<int64_t>(B) * ia.geom.NTS * H),
                                     stream);
    if (e != hipSuccess) return hip_fail(e, "intra kernel launch");
    ia.status_clear = nullptr;
    for (int sgi = 0; sgi < L.segments; ++sgi) {
      sa.geom = seg_geom(sgi);
      sa.W = ia.W; sa.U = ia.U; sa.AQ = ia.AQ; sa.GQ = ia.GQ; sa.LK = ia.LK; sa.GC = ia.GC;
      sa.h0 = (sgi == 0) ? h0 : carry;
      sa.ht = carry;
      if (sgi + 1 < L.segments) {
        set_bufs((sgi + 1) & 1);
        ia.geom = seg_geom(sgi + 1);
        e = kda::launch_overlap(ia, sa, dk, dtq, dtg, out_dt, static_cast<int>(state_grid),
                                static_cast<int>(static_cast<int64_t>(B) * ia.geom.NTS * H), stream);
        if (e != hipSuccess) return hip_fail(e, "overlapped segment launch");
      } else {
        e = kda::launch_state(sa, dk, exact, out_dt, static_cast<int>(state_grid), stream);
        if (e != hipSuccess) return hip_fail(e, "state kernel launch");
      }
    }
    return KDA_OK;
  }
  if (varlen && L.vsegs > 1) {
    // Segmented varlen: per segment an intra launch over its KU units and a
    // state launch that walks each chain's chunks in it, from h0 (a chain's
    // first chunk) or from the state the previous segment left in `carry`.
    float* const vcarry = (ht != nullptr) ? ht : at<float>(ws, L.state);
    for (int sgi = 0; sgi < L.vsegs; ++sgi) {
      G.seg = sgi;
      ia.geom = G;
      sa.geom = G;
      hipError_t e = kda::launch_intra(ia, dk, dtq, dtg, static_cast<int>(static_cast<int64_t>(L.KU) * H), stream);
      if (e != hipSuccess) return hip_fail(e, "intra kernel launch");
      ia.status_clear = nullptr;
      sa.h0 = h0;
      sa.ht = vcarry;
      e = kda::launch_state(sa, dk, exact, out_dt, static_cast<int>(state_grid), stream);
      if (e != hipSuccess) return hip_fail(e, "state kernel launch");
    }
    return KDA_OK;
  }
  for (int sgi = 0; sgi < L.segments; ++sgi) {
    if (!varlen) {
      G.n0 = sgi * L.seg_chunks;
      G.NTS = std::min(L.seg_chunks, G.NT - G.n0);  // 0 only when T == 0: the state kernel then copies h0
    }
    ia.geom = G;
    sa.geom = G;
    const int64_t intra_grid = varlen ? L.units_bound * H : static_cast<int64_t>(B) * G.NTS * H;
    if (intra_grid > 0) {
      hipError_t e = (pro != nullptr) ? kda::launch_intra_prologue(ia, dk, dtg, static_cast<int>(intra_grid), stream)
                                      : kda::launch_intra(ia, dk, dtq, dtg, static_cast<int>(intra_grid), stream);
      if (e != hipSuccess) return hip_fail(e, "intra kernel launch");
      ia.status_clear = nullptr;
    }
    sa.h0 = (sgi == 0) ? h0 : carry;
    sa.ht = (L.segments > 1) ? carry : ht;
    hipError_t e = kda::launch_state(sa, dk, exact, out_dt, static_cast<int>(state_grid), stream);
    if (e != hipSuccess) return hip_fail(e, "state kernel launch");
  }
  if (ia.status_clear != nullptr) {
    // no intra launch ran (T == 0): clear the status word by a kernel
    hipError_t e = kda::launch_copy_or_zero(reinterpret_cast<float*>(status), nullptr, 1, stream);
    if (e != hipSuccess) return hip_fail(e, "status clear launch");
  }
  return KDA_OK;
}

}  // namespace

// ----------------------------------------------------------------------------
// cc_scan adapter kernel: g = log(alpha), beta = mean(beta32 over 32 columns)
// ----------------------------------------------------------------------------
namespace kda {

// Grid-strided: g element by element (consecutive threads, consecutive
// elements), beta one token-head per thread (its 32 columns summed in column
// order).  VEC (every pointer 16-byte aligned): four elements per thread and
// 16-byte non-temporal loads and stores (each value is touched once), the
// beta columns read four at a time and summed in the same order.
template <bool VEC>
__global__ __launch_bounds__(256) void kda_adapt_kernel(AdaptArgs a) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
  const int64_t i0 = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t n = a.n_tok_heads * a.dk;
  if constexpr (VEC) {
    const f4* al = reinterpret_cast<const f4*>(a.alpha);
    f4* go = reinterpret_cast<f4*>(a.g_out);
    for (int64_t i = i0; i < n / 4; i += stride) {
      const f4 x = __builtin_nontemporal_load(al + i);
      __builtin_nontemporal_store(f4{logf(x[0]), logf(x[1]), logf(x[2]), logf(x[3])}, go + i);
    }
    for (int64_t th = i0; th < a.n_tok_heads; th += stride) {
      const f4* b = reinterpret_cast<const f4*>(a.beta32 + th * 32);
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const f4 v = __builtin_nontemporal_load(b + j);
        s += v[0];
        s += v[1];
        s += v[2];
        s += v[3];
      }
      a.beta_out[th] = s * (1.0f / 32.0f);
    }
  } else {
    for (int64_t i = i0; i < n; i += stride) a.g_out[i] = logf(a.alpha[i]);
    for (int64_t th = i0; th < a.n_tok_heads; th += stride) {
      const float* b = a.beta32 + th * 32;
      float s = 0.f;
      for (int j = 0; j < 32; ++j) s += b[j];
      a.beta_out[th] = s * (1.0f / 32.0f);
    }
  }
}

hipError_t launch_adapt(const AdaptArgs& a, hipStream_t s) {
  if (a.n_tok_heads == 0) return hipSuccess;
  const bool vec = a.dk % 4 == 0 &&
                   ((reinterpret_cast<uintptr_t>(a.alpha) | reinterpret_cast<uintptr_t>(a.beta32) |
                     reinterpret_cast<uintptr_t>(a.g_out)) & 15) == 0;
  const int64_t need = (a.n_tok_heads * a.dk / (vec ? 4 : 1) + 255) / 256;
  const int grid = static_cast<int>(need < 8192 ? need : 8192);
  if (vec) hipLaunchKernelGGL(kda_adapt_kernel<true>, dim3(grid), dim3(256), 0, s, a);
  else hipLaunchKernelGGL(kda_adapt_kernel<false>, dim3(grid), dim3(256), 0, s, a);
  return hipGetLastError();
}

// One element (VEC: four, with 16-byte non-temporal loads of the fp32 inputs
// and non-temporal stores; every pointer 16-byte aligned) per thread, and one
// dbeta32 value per thread.
template <bool VEC>
__global__ __launch_bounds__(256) void kda_cc_finish_kernel(CcFinishArgs a) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if constexpr (VEC) {
    if (i < a.n / 4) {
      typedef unsigned int u2v __attribute__((ext_vector_type(2)));
      auto bf4 = [](const f4 x) { return u2v{pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3])}; };
      __builtin_nontemporal_store(bf4(__builtin_nontemporal_load(reinterpret_cast<const f4*>(a.dq32) + i)),
                                  reinterpret_cast<u2v*>(a.dq) + i);
      __builtin_nontemporal_store(bf4(__builtin_nontemporal_load(reinterpret_cast<const f4*>(a.dk32) + i)),
                                  reinterpret_cast<u2v*>(a.dk) + i);
      __builtin_nontemporal_store(bf4(__builtin_nontemporal_load(reinterpret_cast<const f4*>(a.dv32) + i)),
                                  reinterpret_cast<u2v*>(a.dv) + i);
      const f4 g = __builtin_nontemporal_load(reinterpret_cast<const f4*>(a.dg) + i);
      const f4 al = __builtin_nontemporal_load(reinterpret_cast<const f4*>(a.alpha) + i);
      __builtin_nontemporal_store(f4{g[0] / al[0], g[1] / al[1], g[2] / al[2], g[3] / al[3]},
                                  reinterpret_cast<f4*>(a.dalpha) + i);
    }
  } else if (i < a.n) {
    static_cast<u16*>(a.dq)[i] = cvt_bf16(a.dq32[i]);
    static_cast<u16*>(a.dk)[i] = cvt_bf16(a.dk32[i]);
    static_cast<u16*>(a.dv)[i] = cvt_bf16(a.dv32[i]);
    a.dalpha[i] = a.dg[i] / a.alpha[i];
  }
  if (i < a.n_tok_heads * 32) a.dbeta32[i] = a.dbeta[i >> 5] * (1.0f / 32.0f);
}

hipError_t launch_cc_finish(const CcFinishArgs& a, hipStream_t s) {
  const uintptr_t any = reinterpret_cast<uintptr_t>(a.dq32) | reinterpret_cast<uintptr_t>(a.dk32) |
                        reinterpret_cast<uintptr_t>(a.dv32) | reinterpret_cast<uintptr_t>(a.dg) |
                        reinterpret_cast<uintptr_t>(a.alpha) | reinterpret_cast<uintptr_t>(a.dalpha);
  const uintptr_t any8 = reinterpret_cast<uintptr_t>(a.dq) | reinterpret_cast<uintptr_t>(a.dk) |
                         reinterpret_cast<uintptr_t>(a.dv);
  const bool vec = a.n % 4 == 0 && (any & 15) == 0 && (any8 & 7) == 0;
  const int64_t ne = vec ? a.n / 4 : a.n;
  const int64_t n = ne > a.n_tok_heads * 32 ? ne : a.n_tok_heads * 32;
  if (n == 0) return hipSuccess;
  const dim3 grid(static_cast<unsigned>((n + 255) / 256));
  if (vec) hipLaunchKernelGGL(kda_cc_finish_kernel<true>, grid, dim3(256), 0, s, a);
  else hipLaunchKernelGGL(kda_cc_finish_kernel<false>, grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace kda

// ----------------------------------------------------------------------------
// exported entry points
// ----------------------------------------------------------------------------
// Backward workspace: arrays per chunk-head (see kda_internal.h: BwdArgs),
// sized for fp32; the fragment arrays FL, FA, FQ, FW (fp16) serve 16-bit inputs.
struct BwdLayout {
  size_t QG, KL, GCV, AQ, TM, WM, UM, SI, VT, DS, DVT, FL, FA, FQ, FW, FWN, FLT, total;
};

BwdLayout bwd_layout(int B, int T, int H, int d) {
  BwdLayout L{};
  const size_t ch = static_cast<size_t>(B) * ((T + kC - 1) / kC) * H;
  size_t off = 0;
  auto take = [&](size_t bytes) { size_t at = off; off = align_up(off + bytes); return at; };
  const size_t cd = ch * kC * d * 4, cc = ch * kC * kC * 4, dd = ch * d * d * 4;
  L.QG = take(cd);
  L.KL = take(cd);
  L.GCV = take(ch * d * 4);
  L.AQ = take(cc);
  L.TM = take(cc);
  L.WM = take(cd);
  L.UM = take(cd);
  L.SI = take(dd);
  L.VT = take(cd);
  L.DS = take(dd);
  L.DVT = take(cd);
  L.FL = take(ch * 4 * (d / 32) * 1024);
  L.FA = take(ch * 6 * 1024);
  L.FQ = take(ch * (d / 16) * 2 * 1024);
  L.FW = take(ch * (d / 16) * 2 * 1024);
  L.FWN = take(ch * 4 * (d / 32) * 1024);
  L.FLT = take(ch * (d / 16) * 2 * 1024);
  L.total = off;
  return L;
}

int ut_check(const void* a, const void* b, const void* x, int H, int C, int N, int dtype) {
  if (!a || !b || !x) return fail(KDA_ERR_INVALID_ARGUMENT, "null pointer");
  if (H < 1 || N < 1) return fail(KDA_ERR_INVALID_ARGUMENT, "H=%d, N=%d must be >= 1", H, N);
  if (C < 1 || C > 64) return fail(KDA_ERR_UNSUPPORTED, "C=%d: this build solves 1 <= C <= 64", C);
  if (dtype != KDA_DTYPE_F32 && dtype != KDA_DTYPE_BF16)
    return fail(KDA_ERR_INVALID_ARGUMENT, "dtype=%d: a, b, x are F32 or BF16", dtype);
  if (static_cast<int64_t>(H) * ((N + 63) / 64) > 0x7FFFFFFFLL) return fail(KDA_ERR_INVALID_ARGUMENT, "too large");
  return KDA_OK;
}

// ----------------------------------------------------------------------------
// Scratch of kda_chunk_fwd_noalloc: the forward's workspace as a file-scope
// device array, so that entry point allocates nothing.  Each device holds its
// own copy (at its own address) from the library's load until the process
// ends.  In host code `scratch` names a host-side stand-in, not device
// memory: its device address is taken once per device with
// hipGetSymbolAddress and only that pointer is ever handed to kernels.  Calls
// on one device share the array; calls that overlap on one device (two
// streams, two threads) race on it.  No part of it needs clearing between
// calls: the forward writes every workspace word it reads within the call.
// ----------------------------------------------------------------------------
// 256 MiB: the dense config-1 workspace (two segments of 160 MiB budget: 149
// MiB with the carried state), the overlapped config-2 one (two 96 MiB sets:
// 180 MiB) and config 3's least varlen workspace (160 MiB of intra results
// per segment and 64 MiB of carried state: 225 MiB) fit; a larger varlen
// call runs in the segments that fit the scratch.
constexpr size_t kScratchBytes = static_cast<size_t>(256) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of this device's scratch, looked up on the first call on
// the device (with that device current) and kept.
int scratch_for_stream(hipStream_t stream, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (stream != nullptr) {
    int sdev = -1;
    e = hipStreamGetDevice(stream, &sdev);
    if (e != hipSuccess) return hip_fail(e, "hipStreamGetDevice");
    dev = sdev;
  }
  if (dev < 0 || dev >= kMaxDevices) return fail(KDA_ERR_UNSUPPORTED, "device %d: at most %d devices", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    int cur = -1;
    e = hipGetDevice(&cur);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return hip_fail(e, "hipSetDevice");
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    hipError_t e2 = (cur != dev) ? hipSetDevice(cur) : hipSuccess;
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if (e2 != hipSuccess) return hip_fail(e2, "hipSetDevice");
    if (p == nullptr) return fail(KDA_ERR_HIP, "hipGetSymbolAddress(scratch) returned null");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return KDA_OK;
}

extern "C" {

int kda_abi_version(void) { return 102; }

const char* kda_last_error(void) { return g_err; }

size_t kda_chunk_fwd_workspace(int B, int T, int H, int dk, int dv, int chunk, int32_t n_seqs,
                               int in_dtype) {
  if (B < 1 || T < 0 || H < 1 || !dim_ok(dk) || dk != dv || chunk != kC) return 0;
  if (in_dtype < KDA_DTYPE_F32 || in_dtype > KDA_DTYPE_BF16_F32GATES) return 0;
  return ws_layout(B, T, H, dk, dv, n_seqs > 0 ? n_seqs : 0, in_dtype).total;
}

size_t kda_chunk_fwd_workspace_min(int B, int T, int H, int dk, int dv, int chunk, int32_t n_seqs,
                                   int in_dtype) {
  if (B < 1 || T < 0 || H < 1 || !dim_ok(dk) || dk != dv || chunk != kC) return 0;
  if (in_dtype < KDA_DTYPE_F32 || in_dtype > KDA_DTYPE_BF16_F32GATES) return 0;
  const int32_t ns = n_seqs > 0 ? n_seqs : 0;
  const int64_t kmin = ns > 0 ? varlen_min_ku(T, H, dk, dv, ns, in_dtype) : 0;
  return ws_layout(B, T, H, dk, dv, ns, in_dtype, kmin).total;
}

int kda_chunk_fwd(hipStream_t stream, const void* q, const void* k, const void* v,
                  const void* g, const void* beta, const float* h0,
                  const int32_t* cu_seqlens, int32_t n_seqs, void* o, float* ht,
                  int B, int T, int H, int dk, int dv, int chunk, float scale,
                  int in_dtype, int out_dtype, void* workspace, size_t workspace_bytes) {
  g_err[0] = '\0';
  return chunk_fwd_impl(stream, q, k, v, g, beta, h0, cu_seqlens, n_seqs, o, ht, B, T, H, dk, dv,
                        chunk, scale, in_dtype, out_dtype, workspace, workspace_bytes);
}

int kda_chunk_fwd_noalloc(hipStream_t stream, const void* q, const void* k, const void* v,
                          const void* g, const void* beta, const float* h0,
                          const int32_t* cu_seqlens, int32_t n_seqs, void* o, float* ht,
                          int B, int T, int H, int dk, int dv, int chunk, float scale,
                          int in_dtype, int out_dtype) {
  g_err[0] = '\0';
  if (B < 1 || T < 0 || H < 1 || !dim_ok(dk) || dk != dv || chunk != kC ||
      in_dtype < KDA_DTYPE_F32 || in_dtype > KDA_DTYPE_BF16_F32GATES) {
    // the full argument checks with their messages
    return chunk_fwd_impl(stream, q, k, v, g, beta, h0, cu_seqlens, n_seqs, o, ht, B, T, H, dk, dv,
                          chunk, scale, in_dtype, out_dtype, nullptr, 0);
  }
  // the call runs the fastest layout that fits the scratch (a varlen call
  // past it in segments: kda_chunk_fwd with a smaller workspace)
  const size_t need = kda_chunk_fwd_workspace_min(B, T, H, dk, dv, chunk, cu_seqlens != nullptr ? n_seqs : 0,
                                                  in_dtype);
  if (need > kScratchBytes)
    return fail(KDA_ERR_WORKSPACE,
                "kda_chunk_fwd_noalloc: this call needs %zu bytes of scratch, the library's "
                "per-device scratch holds %zu (use kda_chunk_fwd with a caller workspace)",
                need, kScratchBytes);
  void* ws = nullptr;
  if (int rc = scratch_for_stream(stream, &ws)) return rc;
  return chunk_fwd_impl(stream, q, k, v, g, beta, h0, cu_seqlens, n_seqs, o, ht, B, T, H, dk, dv,
                        chunk, scale, in_dtype, out_dtype, ws, kScratchBytes);
}

int kda_chunk_fwd_status(hipStream_t stream, const void* workspace, size_t workspace_bytes,
                         int B, int T, int H, int dk, int dv, int chunk, int32_t n_seqs,
                         int in_dtype, int32_t* flags_out) {
  g_err[0] = '\0';
  if (!flags_out) return fail(KDA_ERR_INVALID_ARGUMENT, "null pointer");
  const size_t need = kda_chunk_fwd_workspace(B, T, H, dk, dv, chunk, n_seqs, in_dtype);
  if (need == 0) return fail(KDA_ERR_INVALID_ARGUMENT, "invalid call arguments");
  const void* ws = workspace;
  if (ws == nullptr) {
    // the call ran through kda_chunk_fwd_noalloc: its workspace is this device's scratch
    void* p = nullptr;
    if (int rc = scratch_for_stream(stream, &p)) return rc;
    ws = p;
    workspace_bytes = kScratchBytes;
  }
  bool fits = false;
  const WsLayout L = ws_layout_for(B, T, H, dk, dv, n_seqs > 0 ? n_seqs : 0, in_dtype, workspace_bytes, &fits);
  if (!fits) return fail(KDA_ERR_WORKSPACE, "workspace does not match");
  int32_t words[2] = {0, 0};
  hipError_t e = hipMemcpyAsync(&words[0], static_cast<const char*>(ws) + L.status, 4, hipMemcpyDeviceToHost, stream);
  if (e == hipSuccess && n_seqs > 0)
    e = hipMemcpyAsync(&words[1], static_cast<const char*>(ws) + L.flags, 4, hipMemcpyDeviceToHost, stream);
  if (e != hipSuccess) return hip_fail(e, "status copy");
  e = hipStreamSynchronize(stream);
  if (e != hipSuccess) return hip_fail(e, "stream synchronize");
  *flags_out = words[0] | words[1];
  return KDA_OK;
}

int kda_varlen_status(hipStream_t stream, const void* workspace, size_t workspace_bytes,
                      int B, int T, int H, int dk, int dv, int chunk, int32_t n_seqs,
                      int in_dtype, int32_t* flags_out) {
  g_err[0] = '\0';
  if (!workspace || !flags_out) return fail(KDA_ERR_INVALID_ARGUMENT, "null pointer");
  if (n_seqs < 1) return fail(KDA_ERR_INVALID_ARGUMENT, "n_seqs=%d must be >= 1", n_seqs);
  const size_t need = kda_chunk_fwd_workspace(B, T, H, dk, dv, chunk, n_seqs, in_dtype);
  bool fits = false;
  const WsLayout L = ws_layout_for(B, T, H, dk, dv, n_seqs, in_dtype, workspace_bytes, &fits);
  if (need == 0 || !fits) return fail(KDA_ERR_WORKSPACE, "workspace does not match");
  hipError_t e = hipMemcpyAsync(flags_out, static_cast<const char*>(workspace) + L.flags, 4,
                                hipMemcpyDeviceToHost, stream);
  if (e != hipSuccess) return hip_fail(e, "flags copy");
  e = hipStreamSynchronize(stream);
  if (e != hipSuccess) return hip_fail(e, "stream synchronize");
  return KDA_OK;
}

int kda_recurrent_step(hipStream_t stream, const void* q, const void* k, const void* v,
                       const void* g, const void* beta, float* state, void* o,
                       int B, int H, int dk, int dv, float scale, int in_dtype, int out_dtype) {
  g_err[0] = '\0';
  if (!q || !k || !v || !g || !beta || !state || !o)
    return fail(KDA_ERR_INVALID_ARGUMENT, "null pointer");
  if (B < 1) return fail(KDA_ERR_INVALID_ARGUMENT, "B=%d must be >= 1", B);
  if (int rc = check_dims(H, dk, dv)) return rc;
  if (in_dtype < KDA_DTYPE_F32 || in_dtype > KDA_DTYPE_F16)
    return fail(KDA_ERR_INVALID_ARGUMENT, "in_dtype=%d: decode takes F32, BF16 or F16", in_dtype);
  if (out_dtype != KDA_DTYPE_F32 && out_dtype != KDA_DTYPE_BF16)
    return fail(KDA_ERR_INVALID_ARGUMENT, "out_dtype=%d: o is emitted as F32 or BF16", out_dtype);
  if (!std::isfinite(scale)) return fail(KDA_ERR_INVALID_ARGUMENT, "scale must be finite");
  if (misaligned(state, 16) || misaligned(v, in_dtype == KDA_DTYPE_F32 ? 16 : 8) ||
      misaligned(o, out_dtype == KDA_DTYPE_F32 ? 16 : 8))
    return fail(KDA_ERR_INVALID_ARGUMENT, "state must be 16-byte aligned, v and o aligned to 4 elements");
  const int64_t grid = static_cast<int64_t>(B) * H;
  if (grid > 0x3FFFFFFFLL) return fail(KDA_ERR_INVALID_ARGUMENT, "B*H too large");
  kda::DecodeArgs a{};
  a.q = q; a.k = k; a.v = v; a.g = g; a.beta = beta;
  a.state = state; a.o = o; a.scale = scale;
  hipError_t e = kda::launch_decode(a, dk, in_dtype, out_dtype == KDA_DTYPE_BF16 ? 1 : 0,
                                    static_cast<int>(grid), stream);
  if (e != hipSuccess) return hip_fail(e, "decode kernel launch");
  return KDA_OK;
}

size_t kda_cc_scan_batched_workspace(int B, int T, int H, int dk, int dv, int chunk) {
  if (B < 1 || T < 0 || H < 1 || !dim_ok(dk) || dk != dv || chunk < 1) return 0;
  const size_t th = static_cast<size_t>(B) * T * H;
  const size_t adapt = align_up(th * dk * 4) + align_up(th * 4);
  return adapt + ws_layout(B, T, H, dk, dv, 0, KDA_DTYPE_BF16_F32GATES).total;
}

size_t kda_cc_scan_workspace(int T, int H, int dk, int dv, int chunk) {
  return kda_cc_scan_batched_workspace(1, T, H, dk, dv, chunk);
}

int kda_cc_scan_batched(hipStream_t stream, const void* q, const void* k, const void* v,
                        const float* alpha, const float* beta32, const float* S_in,
                        float* o, float* S_out, int B, int T, int H, int dk, int dv, int tile, int chunk,
                        void* workspace, size_t workspace_bytes) {
  g_err[0] = '\0';
  if (!q || !k || !v || !alpha || !beta32 || !S_in || !o || !S_out)
    return fail(KDA_ERR_INVALID_ARGUMENT, "null pointer");
  if (B < 1) return fail(KDA_ERR_INVALID_ARGUMENT, "B=%d must be >= 1", B);
  if (T < 0) return fail(KDA_ERR_INVALID_ARGUMENT, "T=%d must be >= 0", T);
  if (chunk < 1) return fail(KDA_ERR_INVALID_ARGUMENT, "chunk=%d must be >= 1", chunk);
  if (T % chunk)
    return fail(KDA_ERR_INVALID_ARGUMENT, "T=%d must be a multiple of the chunk width C=%d", T, chunk);
  if (tile < 1 || tile > 16)
    return fail(KDA_ERR_INVALID_ARGUMENT, "tile=%d outside [1, 16] (the _cc_tile bound)", tile);
  if (int rc = check_dims(H, dk, dv)) return rc;
  const size_t need = kda_cc_scan_batched_workspace(B, T, H, dk, dv, chunk);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(KDA_ERR_WORKSPACE, "workspace of %zu bytes is too small (need %zu)", workspace_bytes, need);
  const size_t th = static_cast<size_t>(B) * T * H;
  const size_t g_bytes = align_up(th * dk * 4);
  const size_t b_bytes = align_up(th * 4);
  // The (B, T, H*d) operands are the [B, T, H, d] layout of the chunked
  // forward; its intra kernel takes the log-decay of alpha (log2 alpha, in
  // its own units) and beta = mean(beta32) (in kda_adapt_kernel's column
  // order; the backward runs that adapter) itself.  The workspace keeps the
  // adapter's g and beta areas unused, so both directions size it the same
  // way.
  void* rest = static_cast<char*>(workspace) + g_bytes + b_bytes;
  return chunk_fwd_impl(stream, q, k, v, alpha, beta32, S_in, nullptr, 0, o, S_out, B, T, H, dk, dv,
                        kC, 1.0f, KDA_DTYPE_BF16_F32GATES, KDA_DTYPE_F32, rest,
                        workspace_bytes - g_bytes - b_bytes, nullptr, true);
}

int kda_cc_scan(hipStream_t stream, const void* q, const void* k, const void* v,
                const float* alpha, const float* beta32, const float* S_in,
                float* o, float* S_out, int T, int H, int dk, int dv, int tile, int chunk,
                void* workspace, size_t workspace_bytes) {
  return kda_cc_scan_batched(stream, q, k, v, alpha, beta32, S_in, o, S_out, 1, T, H, dk, dv, tile, chunk,
                             workspace, workspace_bytes);
}

size_t kda_chunk_bwd_workspace(int B, int T, int H, int dk, int dv, int chunk) {
  if (B < 1 || T < 0 || H < 1 || !dim_ok(dk) || dk != dv || chunk != kC) return 0;
  const size_t total = bwd_layout(B, T, H, dk).total;
  return total > 0 ? total : kAlign;   // 0 is reserved for "bad input"
}

int kda_chunk_bwd(hipStream_t stream, const void* q, const void* k, const void* v, const void* g,
                  const void* beta, const float* h0, const void* dout, const float* dht,
                  float* dq, float* dk, float* dv, float* dg, float* dbeta, float* dh0,
                  int B, int T, int H, int dk_dim, int dv_dim, int chunk, float scale,
                  int in_dtype, int dout_dtype, void* workspace, size_t workspace_bytes) {
  g_err[0] = 0;
  if (B < 1) return fail(KDA_ERR_INVALID_ARGUMENT, "B=%d must be >= 1", B);
  if (T < 0) return fail(KDA_ERR_INVALID_ARGUMENT, "T=%d must be >= 0", T);
  // (with T == 0 the per-token tensors are empty and may be null)
  if (T > 0 && (!q || !k || !v || !g || !beta || !dout))
    return fail(KDA_ERR_INVALID_ARGUMENT, "null input pointer");
  if (T > 0 && (!dq || !dk || !dv || !dg || !dbeta))
    return fail(KDA_ERR_INVALID_ARGUMENT, "null gradient pointer");
  if (int rc = check_dims(H, dk_dim, dv_dim)) return rc;
  if (chunk != kC) return fail(KDA_ERR_UNSUPPORTED, "chunk=%d: this build runs chunk == 64", chunk);
  if (in_dtype < KDA_DTYPE_F32 || in_dtype > KDA_DTYPE_BF16_F32GATES)
    return fail(KDA_ERR_INVALID_ARGUMENT, "in_dtype=%d is not a kda_dtype_t", in_dtype);
  if (dout_dtype != KDA_DTYPE_F32 && dout_dtype != KDA_DTYPE_BF16)
    return fail(KDA_ERR_INVALID_ARGUMENT, "dout_dtype=%d: dout is F32 or BF16", dout_dtype);
  if (!std::isfinite(scale)) return fail(KDA_ERR_INVALID_ARGUMENT, "scale must be finite");
  const int64_t elems = static_cast<int64_t>(B) * T * H * dk_dim;
  if (elems >= (1LL << 40)) return fail(KDA_ERR_INVALID_ARGUMENT, "problem too large");
  const int64_t NT = (T + kC - 1) / kC;
  if (static_cast<int64_t>(B) * NT * H > 0x7FFFFFFFLL) return fail(KDA_ERR_INVALID_ARGUMENT, "too many chunk-heads");
  if (int rc = require_aligned(16, "q, k, v, g, dout, the gradients, the states and the workspace",
                               {q, k, v, g, dout, dq, dk, dv, dg, h0, dht, dh0, workspace}))
    return rc;
  const BwdLayout L = bwd_layout(B, T, H, dk_dim);
  if (!workspace || workspace_bytes < L.total)
    return fail(KDA_ERR_WORKSPACE, "workspace of %zu bytes is too small (need %zu)", workspace_bytes, L.total);
  if (T == 0) {
    // no tokens: the state passes through unchanged, dh0 = dht
    if (dh0 != nullptr) {
      const hipError_t e = kda::launch_copy_or_zero(dh0, dht, static_cast<int64_t>(B) * H * dk_dim * dv_dim, stream);
      if (e != hipSuccess) return hip_fail(e, "dh0 for T == 0");
    }
    return KDA_OK;
  }
  unsigned char* ws = static_cast<unsigned char*>(workspace);
  kda::BwdArgs a{};
  a.B = B; a.T = T; a.H = H; a.NT = static_cast<int>(NT);
  a.q = q; a.k = k; a.v = v; a.g = g; a.beta = beta;
  a.h0 = h0; a.dout = dout; a.dht = dht; a.scale = scale;
  a.dq = dq; a.dk = dk; a.dv = dv; a.dg = dg; a.dbeta = dbeta; a.dh0 = dh0;
  a.QG = reinterpret_cast<float*>(ws + L.QG);
  a.KL = reinterpret_cast<float*>(ws + L.KL);
  a.GCV = reinterpret_cast<float*>(ws + L.GCV);
  a.AQ = reinterpret_cast<float*>(ws + L.AQ);
  a.TM = reinterpret_cast<float*>(ws + L.TM);
  a.WM = reinterpret_cast<float*>(ws + L.WM);
  a.UM = reinterpret_cast<float*>(ws + L.UM);
  a.SI = reinterpret_cast<float*>(ws + L.SI);
  a.VT = reinterpret_cast<float*>(ws + L.VT);
  a.DS = reinterpret_cast<float*>(ws + L.DS);
  a.DVT = reinterpret_cast<float*>(ws + L.DVT);
  a.FL = ws + L.FL;
  a.FA = ws + L.FA;
  a.FQ = ws + L.FQ;
  a.FW = ws + L.FW;
  a.FWN = ws + L.FWN;
  a.FLT = ws + L.FLT;
  const hipError_t e = kda::launch_bwd(a, dk_dim, in_dtype, dout_dtype, stream);
  if (e != hipSuccess) return hip_fail(e, "backward kernel launch");
  return KDA_OK;
}


size_t kda_cc_scan_bwd_batched_workspace(int B, int T, int H, int dk, int dv, int chunk) {
  if (B < 1 || T < 0 || H < 1 || !dim_ok(dk) || dk != dv || chunk < 1) return 0;
  const size_t th = static_cast<size_t>(B) * T * H;
  // g, beta (adapter) + dq, dk, dv, dg fp32 + dbeta fp32 + the dense backward's workspace
  return align_up(th * dk * 4) + align_up(th * 4) + 4 * align_up(th * dk * 4) + align_up(th * 4) +
         kda_chunk_bwd_workspace(B, T, H, dk, dv, kC);
}

size_t kda_cc_scan_bwd_workspace(int T, int H, int dk, int dv, int chunk) {
  return kda_cc_scan_bwd_batched_workspace(1, T, H, dk, dv, chunk);
}

int kda_cc_scan_bwd_batched(hipStream_t stream, const void* q, const void* k, const void* v,
                            const float* alpha, const float* beta32, const float* S_in,
                            const float* d_o, const float* dS, void* dq, void* dk, void* dv,
                            float* dalpha, float* dbeta32, float* dS_in,
                            int B, int T, int H, int dk_dim, int dv_dim, int tile, int chunk,
                            void* workspace, size_t workspace_bytes) {
  g_err[0] = '\0';
  if (B < 1) return fail(KDA_ERR_INVALID_ARGUMENT, "B=%d must be >= 1", B);
  if (!q || !k || !v || !alpha || !beta32 || !S_in || !d_o || !dS || !dq || !dk || !dv || !dalpha ||
      !dbeta32 || !dS_in)
    return fail(KDA_ERR_INVALID_ARGUMENT, "null pointer");
  if (T < 0) return fail(KDA_ERR_INVALID_ARGUMENT, "T=%d must be >= 0", T);
  if (chunk < 1) return fail(KDA_ERR_INVALID_ARGUMENT, "chunk=%d must be >= 1", chunk);
  if (T % chunk)
    return fail(KDA_ERR_INVALID_ARGUMENT, "T=%d must be a multiple of the chunk width C=%d", T, chunk);
  if (tile < 1 || tile > 16)
    return fail(KDA_ERR_INVALID_ARGUMENT, "tile=%d outside [1, 16] (the _cc_tile bound)", tile);
  if (int rc = check_dims(H, dk_dim, dv_dim)) return rc;
  // checked here as well as by the dense backward: the adapter launch comes first
  if (int rc = require_aligned(16, "q, k, v, S_in, do, dS, dS_in and the workspace",
                               {q, k, v, S_in, d_o, dS, dS_in, workspace}))
    return rc;
  const size_t need = kda_cc_scan_bwd_batched_workspace(B, T, H, dk_dim, dv_dim, chunk);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(KDA_ERR_WORKSPACE, "workspace of %zu bytes is too small (need %zu)", workspace_bytes, need);
  const size_t th = static_cast<size_t>(B) * T * H;
  unsigned char* ws = static_cast<unsigned char*>(workspace);
  float* g32 = reinterpret_cast<float*>(ws);
  ws += align_up(th * dk_dim * 4);
  float* b32 = reinterpret_cast<float*>(ws);
  ws += align_up(th * 4);
  float* f[4];
  for (int i = 0; i < 4; ++i) {
    f[i] = reinterpret_cast<float*>(ws);
    ws += align_up(th * dk_dim * 4);
  }
  float* dbeta = reinterpret_cast<float*>(ws);
  ws += align_up(th * 4);
  const size_t rest = workspace_bytes - static_cast<size_t>(ws - static_cast<unsigned char*>(workspace));
  kda::AdaptArgs aa{};
  aa.alpha = alpha; aa.beta32 = beta32; aa.g_out = g32; aa.beta_out = b32;
  aa.n_tok_heads = static_cast<int64_t>(th);
  aa.dk = dk_dim;
  hipError_t e = kda::launch_adapt(aa, stream);
  if (e != hipSuccess) return hip_fail(e, "cc_scan backward adapter launch");
  // the dense backward on the [B, T, H, d] view (the same memory layout)
  const int rc = kda_chunk_bwd(stream, q, k, v, g32, b32, S_in, d_o, dS, f[0], f[1], f[2], f[3], dbeta, dS_in,
                               B, T, H, dk_dim, dv_dim, kC, 1.0f, KDA_DTYPE_BF16_F32GATES, KDA_DTYPE_F32, ws, rest);
  if (rc != KDA_OK) return rc;
  kda::CcFinishArgs fa{};
  fa.dq32 = f[0]; fa.dk32 = f[1]; fa.dv32 = f[2]; fa.dg = f[3]; fa.dbeta = dbeta; fa.alpha = alpha;
  fa.dq = dq; fa.dk = dk; fa.dv = dv; fa.dalpha = dalpha; fa.dbeta32 = dbeta32;
  fa.n = static_cast<int64_t>(th) * dk_dim;
  fa.n_tok_heads = static_cast<int64_t>(th);
  e = kda::launch_cc_finish(fa, stream);
  if (e != hipSuccess) return hip_fail(e, "cc_scan backward finish launch");
  return KDA_OK;
}

int kda_cc_scan_bwd(hipStream_t stream, const void* q, const void* k, const void* v,
                    const float* alpha, const float* beta32, const float* S_in,
                    const float* d_o, const float* dS, void* dq, void* dk, void* dv,
                    float* dalpha, float* dbeta32, float* dS_in,
                    int T, int H, int dk_dim, int dv_dim, int tile, int chunk,
                    void* workspace, size_t workspace_bytes) {
  return kda_cc_scan_bwd_batched(stream, q, k, v, alpha, beta32, S_in, d_o, dS, dq, dk, dv, dalpha, dbeta32,
                                 dS_in, 1, T, H, dk_dim, dv_dim, tile, chunk, workspace, workspace_bytes);
}

int kda_ut_solve(hipStream_t stream, const void* a, const void* b, void* x, int H, int C, int N,
                 int dtype, int transpose) {
  g_err[0] = 0;
  if (int rc = ut_check(a, b, x, H, C, N, dtype)) return rc;
  kda::UtArgs u{};
  u.a = a; u.b = b; u.x = x; u.H = H; u.C = C; u.N = N; u.ntiles = (N + 63) / 64;
  const hipError_t e = kda::launch_ut(u, dtype == KDA_DTYPE_F32 ? 0 : 1, transpose != 0, false, stream);
  if (e != hipSuccess) return hip_fail(e, "ut solve launch");
  return KDA_OK;
}

int kda_ut_solve_bwd(hipStream_t stream, const void* a, const void* x, const void* dx, void* da, void* db,
                     int H, int C, int N, int dtype, int transpose) {
  g_err[0] = 0;
  if (int rc = ut_check(a, dx, db, H, C, N, dtype)) return rc;
  if (!x || !da) return fail(KDA_ERR_INVALID_ARGUMENT, "null pointer");
  kda::UtArgs u{};
  u.a = a; u.b = dx; u.x = db; u.xf = x; u.da = da; u.H = H; u.C = C; u.N = N; u.ntiles = (N + 63) / 64;
  // the adjoint of the forward solve is the transposed solve, and vice versa
  const hipError_t e = kda::launch_ut(u, dtype == KDA_DTYPE_F32 ? 0 : 1, transpose == 0, true, stream);
  if (e != hipSuccess) return hip_fail(e, "ut solve backward launch");
  return KDA_OK;
}

int kda_prologue(hipStream_t stream, const void* qp, const void* kp, const void* vp,
                 const float* wq, const float* wk, const float* wv,
                 const float* bq_in, const float* bk_in, const float* bv_in,
                 float* bq_out, float* bk_out, float* bv_out,
                 void* q, void* k, void* v,
                 int B, int T, int H, int d, int K, int in_dtype, int out_dtype) {
  g_err[0] = 0;
  if (B < 1 || T < 0 || H < 1) return fail(KDA_ERR_INVALID_ARGUMENT, "B=%d, T=%d, H=%d out of range", B, T, H);
  if (!dim_ok(d)) return fail(KDA_ERR_UNSUPPORTED, "d=%d: this build runs d in {64, 128}", d);
  if (K < 1 || K > 8) return fail(KDA_ERR_UNSUPPORTED, "K=%d: conv kernels of 1..8 taps", K);
  if ((in_dtype != KDA_DTYPE_F32 && in_dtype != KDA_DTYPE_BF16) ||
      (out_dtype != KDA_DTYPE_F32 && out_dtype != KDA_DTYPE_BF16))
    return fail(KDA_ERR_INVALID_ARGUMENT, "in_dtype=%d, out_dtype=%d: F32 or BF16", in_dtype, out_dtype);
  if (!wq || !wk || !wv) return fail(KDA_ERR_INVALID_ARGUMENT, "null conv taps");
  if (T > 0 && (!qp || !kp || !vp || !q || !k || !v)) return fail(KDA_ERR_INVALID_ARGUMENT, "null pointer");
  if (static_cast<int64_t>(B) * T * H * 3 / 4 > 0x7FFFFFFFLL) return fail(KDA_ERR_INVALID_ARGUMENT, "too large");
  if (int rc = require_aligned(four_elems(in_dtype) / 2, "qp, kp, vp (two elements)", {qp, kp, vp})) return rc;
  if (int rc = require_aligned(four_elems(out_dtype) / 2, "q, k, v (two elements)", {q, k, v})) return rc;
  kda::PrologueArgs a{};
  a.qp = qp; a.kp = kp; a.vp = vp; a.wq = wq; a.wk = wk; a.wv = wv;
  a.bq_in = bq_in; a.bk_in = bk_in; a.bv_in = bv_in; a.bq_out = bq_out; a.bk_out = bk_out; a.bv_out = bv_out;
  a.q = q; a.k = k; a.v = v; a.B = B; a.T = T; a.H = H; a.K = K;
  const hipError_t e = kda::launch_prologue(a, d, in_dtype == KDA_DTYPE_F32 ? 0 : 1,
                                            out_dtype == KDA_DTYPE_F32 ? 0 : 1, stream);
  if (e != hipSuccess) return hip_fail(e, "prologue launch");
  return KDA_OK;
}

int kda_epilogue(hipStream_t stream, const void* o, const void* gate, void* y, int B, int T, int H, int dv,
                 float eps, int o_dtype, int gate_dtype, int out_dtype) {
  g_err[0] = 0;
  if (B < 1 || T < 0 || H < 1) return fail(KDA_ERR_INVALID_ARGUMENT, "B=%d, T=%d, H=%d out of range", B, T, H);
  if (!dim_ok(dv)) return fail(KDA_ERR_UNSUPPORTED, "dv=%d: this build runs dv in {64, 128}", dv);
  auto ok = [](int dt) { return dt == KDA_DTYPE_F32 || dt == KDA_DTYPE_BF16; };
  if (!ok(o_dtype) || !ok(gate_dtype) || !ok(out_dtype))
    return fail(KDA_ERR_INVALID_ARGUMENT, "dtypes must be F32 or BF16");
  if (!(eps >= 0.f) || !std::isfinite(eps)) return fail(KDA_ERR_INVALID_ARGUMENT, "eps must be finite and >= 0");
  if (T > 0 && (!o || !gate || !y)) return fail(KDA_ERR_INVALID_ARGUMENT, "null pointer");
  if (static_cast<int64_t>(B) * T * H / 4 > 0x7FFFFFFFLL) return fail(KDA_ERR_INVALID_ARGUMENT, "too large");
  if (misaligned(o, four_elems(o_dtype)) || misaligned(gate, four_elems(gate_dtype)) ||
      misaligned(y, four_elems(out_dtype)))
    return fail(KDA_ERR_INVALID_ARGUMENT, "o, gate and y must be aligned to 4 elements");
  kda::EpilogueArgs a{};
  a.o = o; a.gate = gate; a.y = y; a.B = B; a.T = T; a.H = H; a.eps = eps;
  const hipError_t e = kda::launch_epilogue(a, dv, o_dtype == KDA_DTYPE_F32 ? 0 : 1,
                                            gate_dtype == KDA_DTYPE_F32 ? 0 : 1, out_dtype == KDA_DTYPE_F32 ? 0 : 1,
                                            stream);
  if (e != hipSuccess) return hip_fail(e, "epilogue launch");
  return KDA_OK;
}

size_t kda_prologue_bwd_workspace(int B, int T, int H, int d, int K) {
  if (B < 1 || T < 0 || H < 1 || !dim_ok(d) || K < 1 || K > 8) return 0;
  const size_t hd = static_cast<size_t>(H) * d;
  const size_t groups = (static_cast<size_t>(T) + 63) / 64;
  const size_t n = align_up(3 * B * groups * K * hd * 4);   // dw partial sums per 64-row group
  return n > 0 ? n : 256;   // nonzero for T == 0: 0 means unsupported
}

int kda_prologue_bwd(hipStream_t stream, const void* qp, const void* kp, const void* vp,
                     const float* wq, const float* wk, const float* wv,
                     const float* bq_in, const float* bk_in, const float* bv_in,
                     const float* dq, const float* dk, const float* dv,
                     float* dqp, float* dkp, float* dvp, float* dwq, float* dwk, float* dwv,
                     float* dbq, float* dbk, float* dbv,
                     int B, int T, int H, int d, int K, int in_dtype, void* workspace, size_t workspace_bytes) {
  g_err[0] = 0;
  if (B < 1 || T < 0 || H < 1) return fail(KDA_ERR_INVALID_ARGUMENT, "B=%d, T=%d, H=%d out of range", B, T, H);
  if (!dim_ok(d)) return fail(KDA_ERR_UNSUPPORTED, "d=%d: this build runs d in {64, 128}", d);
  if (K < 1 || K > 8) return fail(KDA_ERR_UNSUPPORTED, "K=%d: conv kernels of 1..8 taps", K);
  if (in_dtype != KDA_DTYPE_F32 && in_dtype != KDA_DTYPE_BF16)
    return fail(KDA_ERR_INVALID_ARGUMENT, "in_dtype=%d: projections are F32 or BF16", in_dtype);
  if (!wq || !wk || !wv || !dwq || !dwk || !dwv) return fail(KDA_ERR_INVALID_ARGUMENT, "null conv taps or dw");
  if (T > 0 && (!qp || !kp || !vp || !dq || !dk || !dv || !dqp || !dkp || !dvp))
    return fail(KDA_ERR_INVALID_ARGUMENT, "null pointer");
  if (int rc = require_aligned(four_elems(in_dtype) / 2, "qp, kp, vp (two elements)", {qp, kp, vp})) return rc;
  if (int rc = require_aligned(8, "dq, dk, dv, dqp, dkp, dvp (two elements)", {dq, dk, dv, dqp, dkp, dvp}))
    return rc;
  if (static_cast<int64_t>(B) * T * H * 3 / 4 > 0x7FFFFFFFLL) return fail(KDA_ERR_INVALID_ARGUMENT, "too large");
  const size_t need = kda_prologue_bwd_workspace(B, T, H, d, K);
  if (!workspace || workspace_bytes < need)
    return fail(KDA_ERR_WORKSPACE, "workspace of %zu bytes is too small (need %zu)", workspace_bytes, need);
  kda::PrologueBwdArgs a{};
  a.x[0] = qp; a.x[1] = kp; a.x[2] = vp;
  a.w[0] = wq; a.w[1] = wk; a.w[2] = wv;
  a.bin[0] = bq_in; a.bin[1] = bk_in; a.bin[2] = bv_in;
  a.dy[0] = dq; a.dy[1] = dk; a.dy[2] = dv;
  a.dx[0] = dqp; a.dx[1] = dkp; a.dx[2] = dvp;
  a.dw[0] = dwq; a.dw[1] = dwk; a.dw[2] = dwv;
  a.db[0] = K > 1 ? dbq : nullptr; a.db[1] = K > 1 ? dbk : nullptr; a.db[2] = K > 1 ? dbv : nullptr;
  a.B = B; a.T = T; a.H = H; a.K = K; a.G = (T + 63) / 64;
  a.part = static_cast<float*>(workspace);
  const hipError_t e = kda::launch_prologue_bwd(a, d, in_dtype == KDA_DTYPE_F32 ? 0 : 1, stream);
  if (e != hipSuccess) return hip_fail(e, "prologue backward launch");
  return KDA_OK;
}

int kda_epilogue_bwd(hipStream_t stream, const void* o, const void* gate, const void* dy, float* dout, void* dgate,
                     int B, int T, int H, int dv, float eps, int o_dtype, int gate_dtype, int dy_dtype,
                     int dgate_dtype) {
  g_err[0] = 0;
  if (B < 1 || T < 0 || H < 1) return fail(KDA_ERR_INVALID_ARGUMENT, "B=%d, T=%d, H=%d out of range", B, T, H);
  if (!dim_ok(dv)) return fail(KDA_ERR_UNSUPPORTED, "dv=%d: this build runs dv in {64, 128}", dv);
  auto ok = [](int dt) { return dt == KDA_DTYPE_F32 || dt == KDA_DTYPE_BF16; };
  if (!ok(o_dtype) || !ok(gate_dtype) || !ok(dy_dtype) || !ok(dgate_dtype))
    return fail(KDA_ERR_INVALID_ARGUMENT, "dtypes must be F32 or BF16");
  if (!(eps >= 0.f) || !std::isfinite(eps)) return fail(KDA_ERR_INVALID_ARGUMENT, "eps must be finite and >= 0");
  if (T > 0 && (!o || !gate || !dy || !dout || !dgate)) return fail(KDA_ERR_INVALID_ARGUMENT, "null pointer");
  if (static_cast<int64_t>(B) * T * H / 4 > 0x7FFFFFFFLL) return fail(KDA_ERR_INVALID_ARGUMENT, "too large");
  if (misaligned(o, four_elems(o_dtype)) || misaligned(gate, four_elems(gate_dtype)) ||
      misaligned(dy, four_elems(dy_dtype)) || misaligned(dout, 16) || misaligned(dgate, four_elems(dgate_dtype)))
    return fail(KDA_ERR_INVALID_ARGUMENT, "o, gate, dy, dout and dgate must be aligned to 4 elements");
  kda::EpilogueBwdArgs a{};
  a.o = o; a.gate = gate; a.dy = dy; a.dout = dout; a.dgate = dgate; a.B = B; a.T = T; a.H = H; a.eps = eps;
  auto c = [](int dt) { return dt == KDA_DTYPE_F32 ? 0 : 1; };
  const hipError_t e = kda::launch_epilogue_bwd(a, dv, c(o_dtype), c(gate_dtype), c(dy_dtype), c(dgate_dtype), stream);
  if (e != hipSuccess) return hip_fail(e, "epilogue backward launch");
  return KDA_OK;
}

size_t kda_decode_layer_workspace(int B, int H, int d, int in_dtype) {
  if (B < 1 || H < 1 || !dim_ok(d) || (in_dtype != KDA_DTYPE_F32 && in_dtype != KDA_DTYPE_BF16)) return 0;
  const size_t n = static_cast<size_t>(B) * H * d;
  const size_t es = in_dtype == KDA_DTYPE_F32 ? 4 : 2;
  return 3 * align_up(n * es) + align_up(n * 4);
}

int kda_decode_layer_step(hipStream_t stream, const void* qp, const void* kp, const void* vp,
                          const void* g, const void* beta, const void* gate,
                          const float* wq, const float* wk, const float* wv,
                          float* bq, float* bk, float* bv, float* state, void* y,
                          int B, int H, int d, int K, float scale, float eps, int in_dtype, int out_dtype,
                          void* workspace, size_t workspace_bytes) {
  g_err[0] = 0;
  if (!qp || !kp || !vp || !g || !beta || !gate || !wq || !wk || !wv || !state || !y)
    return fail(KDA_ERR_INVALID_ARGUMENT, "null pointer");
  if (K > 1 && (!bq || !bk || !bv)) return fail(KDA_ERR_INVALID_ARGUMENT, "null conv buffer");
  if (B < 1 || H < 1) return fail(KDA_ERR_INVALID_ARGUMENT, "B=%d, H=%d must be >= 1", B, H);
  if (!dim_ok(d)) return fail(KDA_ERR_UNSUPPORTED, "d=%d: this build runs d in {64, 128}", d);
  if (K < 1 || K > 8) return fail(KDA_ERR_UNSUPPORTED, "K=%d: conv kernels of 1..8 taps", K);
  if ((in_dtype != KDA_DTYPE_F32 && in_dtype != KDA_DTYPE_BF16) ||
      (out_dtype != KDA_DTYPE_F32 && out_dtype != KDA_DTYPE_BF16))
    return fail(KDA_ERR_INVALID_ARGUMENT, "in_dtype=%d, out_dtype=%d: F32 or BF16", in_dtype, out_dtype);
  if (!std::isfinite(scale) || !std::isfinite(eps) || !(eps >= 0.f))
    return fail(KDA_ERR_INVALID_ARGUMENT, "scale and eps must be finite (eps >= 0)");
  if (static_cast<int64_t>(B) * H > 0x3FFFFFFFLL) return fail(KDA_ERR_INVALID_ARGUMENT, "B*H too large");
  if (misaligned(state, 16) || misaligned(y, four_elems(out_dtype)))
    return fail(KDA_ERR_INVALID_ARGUMENT, "state must be 16-byte aligned and y aligned to 4 elements");
  const size_t need = kda_decode_layer_workspace(B, H, d, in_dtype);
  if (!workspace || workspace_bytes < need)
    return fail(KDA_ERR_WORKSPACE, "workspace of %zu bytes is too small (need %zu)", workspace_bytes, need);
  // one fused launch (the workspace is not touched by it)
  kda::DecodeLayerArgs la{};
  la.x[0] = qp; la.x[1] = kp; la.x[2] = vp;
  la.g = g; la.beta = beta; la.gate = gate;
  la.w[0] = wq; la.w[1] = wk; la.w[2] = wv;
  // with K == 1 there are no buffer rows: the kernel reads (and discards) row 0
  // of a stand-in array and writes nothing
  la.buf[0] = K > 1 ? bq : state; la.buf[1] = K > 1 ? bk : state; la.buf[2] = K > 1 ? bv : state;
  la.state = state; la.y = y; la.scale = scale; la.eps = eps; la.B = B; la.H = H; la.K = K;
  const hipError_t e = kda::launch_decode_layer(la, d, in_dtype == KDA_DTYPE_F32 ? 0 : 1,
                                                out_dtype == KDA_DTYPE_F32 ? 0 : 1, stream);
  if (e != hipSuccess) return hip_fail(e, "layer step launch");
  return KDA_OK;
}

}  // extern "C"

namespace {

// The chunked layer forward runs the prologue inside the intra kernel when the
// projections are bf16 and the conv has at most kFusedConvTaps taps;
// otherwise as its own pass into workspace q, k, v.
bool layer_fused(int K, int in_dtype) {
  return (in_dtype == KDA_DTYPE_BF16 || in_dtype == KDA_DTYPE_BF16_F32GATES) && K >= 1 && K <= kda::kFusedConvTaps;
}

struct LayerLayout {
  size_t chunk_ws, o, qkv, total;
};

LayerLayout layer_layout(int B, int T, int H, int d, int K, int in_dtype) {
  LayerLayout L{};
  const size_t n = static_cast<size_t>(B) * T * H * d;
  L.chunk_ws = 0;
  size_t off = align_up(ws_layout(B, T, H, d, d, 0, in_dtype).total);
  L.o = off;
  off += align_up(n * 4);
  L.qkv = off;
  if (!layer_fused(K, in_dtype)) off += 3 * align_up(n * (in_dtype == KDA_DTYPE_F32 ? 4 : 2));
  L.total = off;
  return L;
}

}  // namespace

extern "C" {

size_t kda_layer_fwd_workspace(int B, int T, int H, int d, int K, int in_dtype) {
  if (B < 1 || T < 0 || H < 1 || !dim_ok(d) || K < 1 || K > 8) return 0;
  if (in_dtype < KDA_DTYPE_F32 || in_dtype > KDA_DTYPE_BF16_F32GATES || in_dtype == KDA_DTYPE_F16) return 0;
  return layer_layout(B, T, H, d, K, in_dtype).total;
}

int kda_layer_fwd(hipStream_t stream, const void* qp, const void* kp, const void* vp,
                  const void* g, const void* beta, const void* gate,
                  const float* wq, const float* wk, const float* wv,
                  const float* bq_in, const float* bk_in, const float* bv_in,
                  float* bq_out, float* bk_out, float* bv_out,
                  const float* h0, float* ht, void* y, float* o_out,
                  int B, int T, int H, int d, int K, float scale, float eps,
                  int in_dtype, int gate_dtype, int out_dtype, void* workspace, size_t workspace_bytes) {
  g_err[0] = 0;
  if (B < 1 || T < 0 || H < 1) return fail(KDA_ERR_INVALID_ARGUMENT, "B=%d, T=%d, H=%d out of range", B, T, H);
  if (!dim_ok(d)) return fail(KDA_ERR_UNSUPPORTED, "d=%d: this build runs d in {64, 128}", d);
  if (K < 1 || K > 8) return fail(KDA_ERR_UNSUPPORTED, "K=%d: conv kernels of 1..8 taps", K);
  if (in_dtype != KDA_DTYPE_F32 && in_dtype != KDA_DTYPE_BF16 && in_dtype != KDA_DTYPE_BF16_F32GATES)
    return fail(KDA_ERR_INVALID_ARGUMENT, "in_dtype=%d: F32, BF16 or BF16_F32GATES", in_dtype);
  auto ok = [](int dt) { return dt == KDA_DTYPE_F32 || dt == KDA_DTYPE_BF16; };
  if (!ok(gate_dtype) || !ok(out_dtype))
    return fail(KDA_ERR_INVALID_ARGUMENT, "gate_dtype=%d, out_dtype=%d: F32 or BF16", gate_dtype, out_dtype);
  if (!wq || !wk || !wv) return fail(KDA_ERR_INVALID_ARGUMENT, "null conv taps");
  if (T > 0 && (!qp || !kp || !vp || !g || !beta || !gate || !y))
    return fail(KDA_ERR_INVALID_ARGUMENT, "null input or output pointer");
  if (!std::isfinite(scale) || !std::isfinite(eps) || !(eps >= 0.f))
    return fail(KDA_ERR_INVALID_ARGUMENT, "scale and eps must be finite (eps >= 0)");
  if (static_cast<int64_t>(B) * T * H * 3 / 4 > 0x7FFFFFFFLL) return fail(KDA_ERR_INVALID_ARGUMENT, "too large");
  if (int rc = require_aligned(16, "qp, kp, vp, g, o_out and the workspace", {qp, kp, vp, g, o_out, workspace}))
    return rc;
  if (misaligned(gate, four_elems(gate_dtype)) || misaligned(y, four_elems(out_dtype)))
    return fail(KDA_ERR_INVALID_ARGUMENT, "gate and y must be aligned to 4 elements");
  const LayerLayout L = layer_layout(B, T, H, d, K, in_dtype);
  if (!workspace || workspace_bytes < L.total)
    return fail(KDA_ERR_WORKSPACE, "workspace of %zu bytes is too small (need %zu)", workspace_bytes, L.total);
  unsigned char* ws = static_cast<unsigned char*>(workspace);
  float* o = o_out != nullptr ? o_out : reinterpret_cast<float*>(ws + L.o);   // the scan's fp32 output
  const size_t chunk_bytes = L.o;
  kda::PrologueArgs p{};
  p.qp = qp; p.kp = kp; p.vp = vp; p.wq = wq; p.wk = wk; p.wv = wv;
  p.bq_in = bq_in; p.bk_in = bk_in; p.bv_in = bv_in; p.bq_out = bq_out; p.bk_out = bk_out; p.bv_out = bv_out;
  p.B = B; p.T = T; p.H = H; p.K = K;
  const int pdt = in_dtype == KDA_DTYPE_F32 ? 0 : 1;
  hipError_t e;
  if (layer_fused(K, in_dtype)) {
    FusedPrologue fp{{wq, wk, wv}, {bq_in, bk_in, bv_in}, K};
    const int rc = chunk_fwd_impl(stream, qp, kp, vp, g, beta, h0, nullptr, 0, o, ht, B, T, H, d, d, 64, scale,
                                  in_dtype, KDA_DTYPE_F32, ws, chunk_bytes, &fp);
    if (rc != KDA_OK) return rc;
    // the buffers are rewritten after every read of the old ones
    e = kda::launch_prologue_buffers(p, d, pdt, stream);
    if (e != hipSuccess) return hip_fail(e, "layer conv buffer launch");
  } else {
    const size_t n = static_cast<size_t>(B) * T * H * d;
    const size_t es = in_dtype == KDA_DTYPE_F32 ? 4 : 2;
    p.q = ws + L.qkv;
    p.k = ws + L.qkv + align_up(n * es);
    p.v = ws + L.qkv + 2 * align_up(n * es);
    e = kda::launch_prologue(p, d, pdt, pdt, stream);
    if (e != hipSuccess) return hip_fail(e, "layer prologue launch");
    const int rc = chunk_fwd_impl(stream, p.q, p.k, p.v, g, beta, h0, nullptr, 0, o, ht, B, T, H, d, d, 64, scale,
                                  in_dtype, KDA_DTYPE_F32, ws, chunk_bytes);
    if (rc != KDA_OK) return rc;
  }
  kda::EpilogueArgs ep{};
  ep.o = o; ep.gate = gate; ep.y = y; ep.B = B; ep.T = T; ep.H = H; ep.eps = eps;
  e = kda::launch_epilogue(ep, d, 0, gate_dtype == KDA_DTYPE_F32 ? 0 : 1, out_dtype == KDA_DTYPE_F32 ? 0 : 1, stream);
  if (e != hipSuccess) return hip_fail(e, "layer epilogue launch");
  return KDA_OK;
}

}  // extern "C"
