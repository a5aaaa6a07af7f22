// varlen scheduling: validated cu_seqlens, chunk offsets, longest-first order.
#include "kda_common.h"
#include "kda_internal.h"

namespace kda {

constexpr int kCv = 64;

// ----------------------------------------------------------------------------
// varlen preparation: clamp cu_seqlens, chunk offsets, longest-first order
// ----------------------------------------------------------------------------
__global__ __launch_bounds__(1024)
void kda_varlen_prep_kernel(const int32_t* cu, int N, int T, int32_t* cu_clamped,
                            int32_t* chunk_off, int32_t* n_units, int32_t* order,
                            int32_t* flags, int32_t* pos_off, int32_t* seg_pos, int KU, int n_seg) {
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
    if (i < N) cnt = (cu_clamped[i + 1] - cu_clamped[i] + kCv - 1) / kCv;
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
  // longest-first order (bitonic sort of (-len, idx) over the next power of
  // two >= N); identity for large N
  if (N <= 2048) {
    int P = 2;
    while (P < N) P <<= 1;
    for (int i = tid; i < P; i += 1024) {
      if (i < N) {
        const int64_t len = cu_clamped[i + 1] - cu_clamped[i];
        keys[i] = ((int64_t)(0x7FFFFFFF - len) << 32) | (uint32_t)i;
      } else {
        keys[i] = INT64_MAX;
      }
    }
    __syncthreads();
    for (int k = 2; k <= P; k <<= 1) {
      for (int j = k >> 1; j > 0; j >>= 1) {
        for (int i = tid; i < P; i += 1024) {
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
  if (pos_off == nullptr) return;
  // Segmented calls (N <= 2048, so keys[] holds the lengths longest-first):
  // position-major unit numbering.  cnt(p), the sequences with more than p
  // chunks, are ranks 0 .. cnt(p) - 1; pos_off is its exclusive scan over
  // the positions 0 .. n_pos (n_pos = the longest sequence's chunks).
  auto len_of_rank = [&](int r) -> int { return 0x7FFFFFFF - (int)(keys[r] >> 32); };
  const int n_pos = (N > 0) ? (len_of_rank(0) + kCv - 1) / kCv : 0;
  if (tid == 0) carry = 0;
  __syncthreads();
  for (int base = 0; base <= n_pos; base += 1024) {
    const int p = base + tid;
    int cnt = 0;
    if (p < n_pos) {
      // first rank whose length is at most 64 p (lengths non-increasing in rank)
      int lo = 0, hi = N;
      while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (len_of_rank(mid) > kCv * p) lo = mid + 1; else hi = mid;
      }
      cnt = lo;
    }
    scan[tid] = cnt;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {
      int t = (tid >= off) ? scan[tid - off] : 0;
      __syncthreads();
      scan[tid] += t;
      __syncthreads();
    }
    if (p <= n_pos) pos_off[p] = carry + scan[tid] - cnt;
    __syncthreads();
    if (tid == 1023) carry += scan[1023];
    __syncthreads();
  }
  // position and rank of each segment's first unit s * KU (s = 0 .. n_seg);
  // past the last unit: (n_pos, 0)
  const int nu = carry;
  for (int sg = tid; sg <= n_seg; sg += 1024) {
    const int64_t U = static_cast<int64_t>(sg) * KU;
    int P = n_pos, R = 0;
    if (U < nu) {
      int lo = 0, hi = n_pos - 1;   // largest p with pos_off[p] <= U
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (pos_off[mid] <= U) lo = mid; else hi = mid - 1;
      }
      P = lo;
      R = static_cast<int>(U - pos_off[lo]);
    }
    seg_pos[2 * sg] = P;
    seg_pos[2 * sg + 1] = R;
  }
}

hipError_t launch_varlen_prep(const int32_t* cu, int N, int T, int32_t* cu_clamped,
                              int32_t* chunk_off, int32_t* n_units, int32_t* order,
                              int32_t* flags, int32_t* pos_off, int32_t* seg_pos, int KU, int n_seg,
                              hipStream_t s) {
  hipLaunchKernelGGL(kda_varlen_prep_kernel, dim3(1), dim3(1024), 0, s, cu, N, T, cu_clamped,
                     chunk_off, n_units, order, flags, pos_off, seg_pos, KU, n_seg);
  return hipGetLastError();
}

}  // namespace kda
