// Internal argument structs and launchers shared by the KDA translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kda {

// Geometry of one chunked call.  Dense: B sequences of T tokens (cu == null).
// Varlen: one packed stream of T tokens split by cu_seqlens into N sequences.
struct Geom {
  int B, T, H;
  int NT;                       // dense: chunks per sequence
  int n0;                       // dense: first chunk of the segment this launch covers
  int NTS;                      // dense: chunks in that segment (workspace units per sequence)
  int N;                        // number of sequences (dense: B)
  const int32_t* cu;            // original cu_seqlens (varlen) or null
  const int32_t* cu_clamped;    // validated copy (varlen)
  const int32_t* chunk_off;     // [N+1] first chunk unit of each sequence (varlen)
  const int32_t* n_units;       // total chunk units (varlen, device)
  const int32_t* order;         // longest-first sequence order (varlen) or null
  // Segmented varlen calls (pos_off non-null).  Units are numbered
  // position-major: every sequence's chunk p precedes every sequence's chunk
  // p + 1, and at position p the sequences of longest-first rank 0 ..
  // cnt(p) - 1 (the ones with more than p chunks) hold units pos_off[p] +
  // rank.  A launch covers units [seg * KU, (seg + 1) * KU); its workspace
  // slot of unit u is u - seg * KU.  seg_pos[2 s], seg_pos[2 s + 1] are the
  // position and rank of unit s * KU (the first unit of segment s).
  const int32_t* pos_off;       // [n_pos + 1], device (prep kernel)
  const int32_t* seg_pos;       // [2 (n_seg + 1)], device (prep kernel)
  int seg;                      // segment of this launch
  int KU;                       // units per segment
};

struct IntraArgs {
  Geom geom;
  const void* q;
  const void* k;
  const void* v;
  const void* g;
  const void* beta;
  float scale;
  void* W;    // per chunk-head, fragment order (see kda_chunk.hip)
  void* U;
  void* AQ;
  void* GQ;
  void* LK;
  float* GC;
  // Fused prologue (K > 0): q, k, v are the raw projections qp, kp, vp and
  // the kernel applies the short conv (taps cw[t] [K][H*dk] fp32, history of
  // each sequence's first chunk cb[t] [N][K-1][H*dk] fp32 or null = zeros),
  // swish and, for q and k, the L2 norm before everything else.
  const float* cw[3];
  const float* cb[3];
  int K;
  int* status_clear;   // non-null: the launch zeroes the call's status word
  int total;           // chunk-heads of the launch (overlapped-segment launch only)
  // cc_scan operands (fp32 gates only): g holds alpha (the decay factor; the
  // kernel takes log2(alpha) by the hardware logarithm, the log-decay in the
  // base-2 units it works in) and beta holds beta32 [T*H][32] (the kernel
  // takes the mean of the 32 columns, summed in column order)
  int gates_alpha;
};

struct StateArgs {
  Geom geom;
  const void* W;
  const void* U;
  const void* AQ;
  const void* GQ;
  const void* LK;
  const float* GC;
  const float* h0;
  void* o;
  float* ht;
  // non-null (16-bit inputs): bit kStatusNonFinite is set when an o or final
  // state value of the call is not finite
  int* status;
};

// status word of a chunked forward call: a non-finite o or final state value
// (an fp16 operand out of range, or non-finite inputs)
constexpr int kStatusNonFinite = 1 << 16;

struct DecodeArgs {
  const void* q;
  const void* k;
  const void* v;
  const void* g;
  const void* beta;
  float* state;
  void* o;
  float scale;
};

struct AdaptArgs {
  const float* alpha;
  const float* beta32;
  float* g_out;
  float* beta_out;
  int64_t n_tok_heads;  // T * H
  int dk;
};

// Chunked backward (dense inputs; workspace arrays row-major per chunk-head
// ch = (b * NT + n) * H + h, fp32, or for 16-bit inputs fp16 where kda_bwd.hip
// says so; the F* arrays, written and read only with 16-bit inputs, are fp16
// MFMA A fragments: lane (r = l & 15, gq = l >> 4) of K step s holds M index
// 16 m + r and K indices 32 s + 4 gq + (e & 3) + 16 (e >> 2), e = 0..7).
struct BwdArgs {
  int B, T, H, NT;
  const void* q;
  const void* k;
  const void* v;
  const void* g;
  const void* beta;
  const float* h0;      // [B,H,dk,dv] or null
  const void* dout;     // cotangent of o, [B,T,H,dv] (fp32 or bf16)
  const float* dht;     // cotangent of the final state, [B,H,dk,dv] or null
  float scale;
  float* dq;            // [B,T,H,dk]
  float* dk;
  float* dv;            // [B,T,H,dv]
  float* dg;            // [B,T,H,dk]
  float* dbeta;         // [B,T,H]
  float* dh0;           // [B,H,dk,dv] or null
  float* QG;            // [ch][C][dk] gamma * q (scaled)
  float* KL;            // [ch][C][dk] lambda * k
  float* GCV;           // [ch][dk]    gamma_C
  float* AQ;            // [ch][C][C]  Aqk
  float* TM;            // [ch][C][C]  (I + L)^-1
  float* WM;            // [ch][C][dk]
  float* UM;            // [ch][C][dv]
  float* SI;            // [ch][dk][dv] state entering the chunk
  float* VT;            // [ch][C][dv] v~
  float* DS;            // [ch][dk][dv] cotangent of the state leaving the chunk
  float* DVT;           // [ch][C][dv] cotangent of v~
  void* FL;             // [ch][4][dk/32][64][8]  lambda k (M rows, K channels)
  void* FA;             // [ch][6][64][8]         Aqk^T (M key rows, K query rows): (key tile, K step)
                        //                        00 01 10 11 21 31 (the others are zero)
  void* FQ;             // [ch][dk/16][2][64][8]  (gamma q)^T (M channels, K rows)
  void* FW;             // [ch][dk/16][2][64][8]  W^T (M channels, K rows)
  void* FWN;            // [ch][4][dk/32][64][8]  W (M rows, K channels)
  void* FLT;            // [ch][dk/16][2][64][8]  (lambda k)^T (M channels, K rows)
};

// Standalone unit-triangular solve (kda_ut.hip); a [H][C][C], b/x/xf [H][C][N].
struct UtArgs {
  const void* a;
  const void* b;    // right-hand side (the cotangent dX in the backward rule)
  void* x;          // solution (dB in the backward rule)
  const void* xf;   // backward rule: the forward solution X
  void* da;         // backward rule: dA (strict lower), else unused
  int H, C, N, ntiles;
};

// Prologue / epilogue around the chunked kernels (kda_prologue.hip).
struct PrologueArgs {
  const void* qp;          // [B,T,H*d] projections (fp32 or bf16)
  const void* kp;
  const void* vp;
  const float* wq;         // [K, H*d] depthwise conv taps, w[i] weights x[t-i]
  const float* wk;
  const float* wv;
  const float* bq_in;      // [B, K-1, H*d] history rows, oldest first, or null (zeros)
  const float* bk_in;
  const float* bv_in;
  float* bq_out;           // last K-1 inputs after this call, or null
  float* bk_out;
  float* bv_out;
  void* q;                 // [B,T,H,d] outputs (fp32 or bf16)
  void* k;
  void* v;
  int B, T, H, K;
};

struct EpilogueArgs {
  const void* o;           // [B,T,H,dv]
  const void* gate;        // [B,T,H*dv] gate logits
  void* y;                 // [B,T,H*dv]
  int B, T, H;
  float eps;
};

// Backward of the prologue: cotangents dq, dk, dv [B,T,H,d] fp32 of its
// outputs -> dx (projections), dw (conv taps), db (incoming buffers).
struct PrologueBwdArgs {
  const void* x[3];        // qp, kp, vp [B,T,H*d] (fp32 or bf16)
  const float* w[3];       // [K, H*d]
  const float* bin[3];     // [B, K-1, H*d] or null (zeros)
  const float* dy[3];      // dq, dk, dv [B,T,H*d] fp32
  float* dx[3];            // [B,T,H*d] fp32
  float* dw[3];            // [K, H*d] fp32
  float* db[3];            // [B, K-1, H*d] fp32 or null (not wanted)
  float* part;             // workspace: [3][B * G][K][H*d] fp32, dw partial sums (G groups of 64 rows)
  int B, T, H, K, G;
};

struct EpilogueBwdArgs {
  const void* o;           // [B,T,H,dv]
  const void* gate;        // [B,T,H*dv] gate logits
  const void* dy;          // [B,T,H*dv]
  float* dout;             // [B,T,H,dv] fp32
  void* dgate;             // [B,T,H*dv]
  int B, T, H;
  float eps;
};

hipError_t launch_prologue(const PrologueArgs& a, int d, int in_dt, int out_dt, hipStream_t s);
hipError_t launch_prologue_bwd(const PrologueBwdArgs& a, int d, int in_dt, hipStream_t s);
hipError_t launch_epilogue_bwd(const EpilogueBwdArgs& a, int d, int o_dt, int g_dt, int dy_dt, int dg_dt,
                               hipStream_t s);
// only the conv buffer update of launch_prologue (the last K-1 inputs)
hipError_t launch_prologue_buffers(const PrologueArgs& a, int d, int in_dt, hipStream_t s);
hipError_t launch_epilogue(const EpilogueArgs& a, int d, int o_dt, int g_dt, int y_dt, hipStream_t s);
hipError_t launch_bwd(const BwdArgs& a, int d, int in_dtype, int do_dtype, hipStream_t s);
hipError_t launch_ut(const UtArgs& a, int dtype, bool transpose, bool with_da, hipStream_t s);
// dst[0..n) = src (or 0 when src is null), by a kernel (no memset/memcpy node)
hipError_t launch_copy_or_zero(float* dst, const float* src, int64_t n, hipStream_t s);
hipError_t launch_intra(const IntraArgs& a, int d, int dtq, int dtg, int grid, hipStream_t s);
// the intra kernel with the fused prologue (a.K in [1, kFusedConvTaps], bf16 q, k, v)
hipError_t launch_intra_prologue(const IntraArgs& a, int d, int dtg, int grid, hipStream_t s);
constexpr int kFusedConvTaps = 4;
hipError_t launch_state(const StateArgs& a, int d, bool exact, int out_dt, int grid, hipStream_t s);
// state scan of one segment (n_state workgroups of the 32-column state
// kernel's grid) and intra-chunk work of the next (intra_units chunk-heads)
// in one launch; fp16 operands, no fused prologue
hipError_t launch_overlap(const IntraArgs& ia, const StateArgs& sa, int d, int dtq, int dtg, int out_dt,
                          int n_state, int intra_units, hipStream_t s);
// varlen preparation; pos_off / seg_pos non-null (segmented calls, N <= 2048):
// also the position-major unit tables of Geom for segments of KU units
// (n_seg segments)
hipError_t launch_varlen_prep(const int32_t* cu, int N, int T, int32_t* cu_clamped,
                              int32_t* chunk_off, int32_t* n_units, int32_t* order,
                              int32_t* flags, int32_t* pos_off, int32_t* seg_pos, int KU, int n_seg,
                              hipStream_t s);
hipError_t launch_decode(const DecodeArgs& a, int d, int dt, int out_dt, int grid, hipStream_t s);

// One decode token of the whole layer in one launch: short conv (buffers
// shifted in place), swish, L2 norm of q and k, the delta-rule step on the
// fp32 state in place, head-wise RMSNorm x sigmoid gate.
struct DecodeLayerArgs {
  const void* x[3];        // qp, kp, vp [B, H*d]
  const void* g;           // [B, H, d] log decay
  const void* beta;        // [B, H]
  const void* gate;        // [B, H*d] logits
  const float* w[3];       // conv taps [K, H*d]
  float* buf[3];           // conv buffers [B, K-1, H*d] (updated in place)
  float* state;            // [B, H, d, d]
  void* y;                 // [B, H*d]
  float scale, eps;
  int B, H, K;
};
hipError_t launch_decode_layer(const DecodeLayerArgs& a, int d, int dt, int out_dt, hipStream_t s);
hipError_t launch_adapt(const AdaptArgs& a, hipStream_t s);

// cc_scan backward outputs from the dense backward's fp32 results: dq, dk, dv
// rounded to bf16 (the primal dtype), dalpha = dg / alpha (g = log alpha),
// dbeta32 = dbeta / 32 on each of the 32 columns (beta = their mean).
struct CcFinishArgs {
  const float* dq32;
  const float* dk32;
  const float* dv32;
  const float* dg;
  const float* dbeta;
  const float* alpha;
  void* dq;                // bf16
  void* dk;
  void* dv;
  float* dalpha;
  float* dbeta32;
  int64_t n;               // T * H * d
  int64_t n_tok_heads;     // T * H
};
hipError_t launch_cc_finish(const CcFinishArgs& a, hipStream_t s);

}  // namespace kda
