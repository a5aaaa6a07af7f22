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
};

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

hipError_t launch_intra(const IntraArgs& a, int d, int dtq, int dtg, int grid, hipStream_t s);
hipError_t launch_state(const StateArgs& a, int d, bool exact, int out_dt, int grid, hipStream_t s);
hipError_t launch_varlen_prep(const int32_t* cu, int N, int T, int32_t* cu_clamped,
                              int32_t* chunk_off, int32_t* n_units, int32_t* order,
                              int32_t* flags, hipStream_t s);
hipError_t launch_decode(const DecodeArgs& a, int d, int dt, int out_dt, int grid, hipStream_t s);
hipError_t launch_adapt(const AdaptArgs& a, hipStream_t s);

}  // namespace kda
