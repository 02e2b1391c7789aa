// Host-side entry points of the kernels, shared between the C ABI (capi.cpp) and the kernel sources.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "gdn_common.h"

namespace qbgdn {

// A validated call: the descriptor resolved into sizes and the packed-sequence table.
struct Problem {
  int B, T, Hk, Hv, Dk, Dv;
  int in_bf16;   // 1: q, k, v, beta are bfloat16; 0: float32
  int out_bf16;  // 1: y, dy, dq, dk, dv, dbeta are bfloat16; 0: float32
  int g_is_log;
  int N;         // state count: B, or the number of packed sequences
  int64_t BT;    // tokens
  int64_t NC;    // chunk slots
  SeqTable tab;
};

// Forward pointers (device). s0, s_out, ckpt may be null.
struct FwdPtrs {
  const void* q;
  const void* k;
  const void* v;
  const float* g;
  const void* beta;
  const float* s0;
  void* y;
  float* s_out;
  float* ckpt;
  float* rows = nullptr;  // the state after every token [tokens, Hv, Dv, Dk] (recurrent design only); may be null
};

// Backward pointers (device). ds_out, ds0 may be null.
struct BwdPtrs {
  const void* q;
  const void* k;
  const void* v;
  const float* g;
  const void* beta;
  const float* ckpt;
  const void* dy;
  const float* ds_out;
  void* dq;
  void* dk;
  void* dv;
  float* dg;
  void* dbeta;
  float* ds0;
};

// Optional per-launch events (qb_gdn_desc.trace_events): mark() before each kernel launch and once after the last.
struct Tracer {
  void** ev = nullptr;
  int n = 0;
  int i = 0;
  hipStream_t s = nullptr;
  void mark() {
    if (ev && i < n) (void)hipEventRecord(static_cast<hipEvent_t>(ev[i++]), s);
  }
};

// Design 1: recurrent, one state row per 16 lanes.
const char* rec_supports(const Problem& p);  // null when supported, else why not
size_t rec_ckpt_bytes(const Problem& p);
size_t rec_workspace_bytes(const Problem& p);
extern const char* const kRecFwdLaunches;  // comma-separated kernel names, in launch order
extern const char* const kRecBwdLaunches;
hipError_t rec_fwd(const Problem& p, const FwdPtrs& a, void* ws, hipStream_t s, Tracer& tr);
hipError_t rec_bwd(const Problem& p, const BwdPtrs& a, void* ws, hipStream_t s, Tracer& tr);

// Design 1 past Dk = 256 (rec_wide.hip): one wave per state row, rows per block for the forward and the backward
// (the backward's is the row-block granularity of its partials), the backward's per-row scratch, and the kernels.
int rec_wide_fwd_rows(int Dk);
int rec_wide_bwd_rows(int Dk);
size_t rec_wide_scratch_bytes(const Problem& p);
template <typename InT, typename OutT>
hipError_t rec_wide_fwd(const Problem& p, const FwdPtrs& ptrs, hipStream_t s);
template <typename InT, typename OutT>
hipError_t rec_wide_bwd(const Problem& p, const BwdPtrs& ptrs, float* dq_part, float* dk_part, float* dg_part,
                        float* db_part, float* scratch, int nblk, hipStream_t s);

// Design 2: chunkwise WY/UT form on MFMA.
const char* chunk_supports(const Problem& p);
size_t chunk_ckpt_bytes(const Problem& p);
size_t chunk_workspace_bytes(const Problem& p);
extern const char* const kChunkFwdLaunches;
extern const char* const kChunkBwdLaunches;
hipError_t chunk_fwd(const Problem& p, const FwdPtrs& a, void* ws, hipStream_t s, Tracer& tr);
// The layer's prologue fused into the chunked forward (qb_gdn_fwd_prologue): its raw inputs and its outputs, which
// the forward writes and then runs on (a.q, a.k, a.g, a.beta must be q, k, log_decay, beta below).
struct PrologueIn {
  const void* q_raw;
  const void* k_raw;
  const void* a;
  const void* b;
  const float* a_log;
  const float* dt_bias;
  float scale_q, scale_k;  // 1/Dk and Dk^-1/2 in the activation dtype
  void* q;
  void* k;
  void* beta;
  float* log_decay;
};
hipError_t chunk_fwd_prologue(const Problem& p, const PrologueIn& pro, const FwdPtrs& a, void* ws, hipStream_t s,
                              Tracer& tr);
// The layer's prologue backward fused into the chunked backward (qb_gdn_bwd_prologue): the raw inputs and the
// prologue's cotangents, which replace those of q, k, g and beta (a.dq, a.dk, a.dg, a.dbeta are not written).
struct PrologueGradIn {
  const void* q_raw;
  const void* k_raw;
  const void* a;
  const void* b;
  const float* a_log;
  const float* dt_bias;
  float scale_q, scale_k;
  void* dq_raw;
  void* dk_raw;
  void* da;
  void* db;
  float* da_log;
  float* ddt_bias;
};
hipError_t chunk_bwd_prologue(const Problem& p, const PrologueGradIn& pro, const BwdPtrs& a, void* ws,
                              hipStream_t s, Tracer& tr);
hipError_t chunk_bwd(const Problem& p, const BwdPtrs& a, void* ws, hipStream_t s, Tracer& tr);

}  // namespace qbgdn
