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
  float* dqk_part;  // workspace, short sequences: per (chunk slot, value head) dq and dk [64][128] float32, or null
  ChunkLayout lay;
  int Hk, Hv, Dv, g_is_log;
  int nblk;  // state-row blocks of a head in the state passes: Dv / 16 or Dv / 32
  int N;     // sequences
  SeqTable tab;
  // The layer's prologue fused into chunk_prep (qb_gdn_fwd_prologue): the raw inputs, and the prologue's outputs,
  // which prep writes and the later kernels read as q, k, g (the log-decay) and beta.
  struct Prologue {
    const bf16_t* q_raw;
    const bf16_t* k_raw;
    const bf16_t* a;
    const bf16_t* b;
    const float* a_log;
    const float* dt_bias;
    float scale_q, scale_k;
    bf16_t* q;
    bf16_t* k;
    bf16_t* beta;
    float* log_decay;
    // The fused backward (chunk_bwd_grads): the cotangents of a and b, and per (chunk slot, value head) the sums
    // of the dA_log and ddt_bias terms [NC][Hv][2]. dq_raw and dk_raw go to dq and dk.
    bf16_t* da;
    bf16_t* db;
    float* part;
  } pro;
};

hipError_t launch_chunk_prep(const ChunkArgs& a, hipStream_t s, bool fused_prologue = false);
hipError_t launch_chunk_fwd(const ChunkArgs& a, bool out_bf16, hipStream_t s);
hipError_t launch_chunk_bwd_state(const ChunkArgs& a, bool out_bf16, hipStream_t s);
hipError_t launch_chunk_dqk_sum(const ChunkArgs& a, bool out_bf16, hipStream_t s, bool fused_prologue);
hipError_t launch_chunk_bwd_grads(const ChunkArgs& a, bool out_bf16, hipStream_t s, bool fused_prologue = false);
hipError_t launch_chunk_gate_sums(const ChunkArgs& a, float* da_log, float* ddt_bias, hipStream_t s);
hipError_t launch_chunk_dgfix(const ChunkArgs& a, bool out_bf16, hipStream_t s);

}  // namespace qbgdn
