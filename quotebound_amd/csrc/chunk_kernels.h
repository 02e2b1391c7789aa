// Arguments and launchers of the chunked design's kernels (chunk_prep.hip, chunk_fwd.hip, chunk_bwd_state.hip,
// chunk_bwd_grads.hip, chunk_dgfix.hip); chunk.hip sequences them.
#pragma once
#include "chunk_common.h"

namespace qbgdn {

struct ChunkArgs {
  const bf16_t* q;
  const bf16_t* k;
  const bf16_t* v;
  const bf16_t* beta;
  const float* g;
  const float* s0;
  void* y;
  float* s_out;
  float* ckpt;   // chunk-start states (may be null in a forward without backward)
  Tile* tiles;   // per (slot, value head): inside ckpt after the states, or in the workspace
  const void* dy;
  const float* ds_out;
  void* dq;
  void* dk;
  void* dv;
  float* dg;
  void* dbeta;
  float* ds0;
  float* dsend;  // workspace: cotangent of each chunk's end state
  ChunkLayout lay;
  int Hk, Hv, Dv, g_is_log;
  int nblk;  // Dv / 16 state-row blocks
  int N;     // sequences
  SeqTable tab;
};

hipError_t launch_chunk_prep(const ChunkArgs& a, hipStream_t s);
hipError_t launch_chunk_fwd(const ChunkArgs& a, bool out_bf16, hipStream_t s);
hipError_t launch_chunk_bwd_state(const ChunkArgs& a, bool out_bf16, hipStream_t s);
hipError_t launch_chunk_bwd_grads(const ChunkArgs& a, bool out_bf16, hipStream_t s);
hipError_t launch_chunk_dgfix(const ChunkArgs& a, bool out_bf16, hipStream_t s);

}  // namespace qbgdn
