// The layer's pointwise neighbours of the recurrence (neighbours.hip): the q/k normalisation, beta and log-decay
// before it, the gated RMSNorm after it, and their backward.
#pragma once
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace qbgdn {

struct NbProblem {
  int64_t BT;  // tokens
  int Hk, Hv, Dk, Dv;
  int bf16;    // activations in bfloat16 (else float32)
  float scale_q, scale_k;  // 1/Dk and Dk^-1/2, rounded to the activation dtype
};

struct NbPrologue {
  const void* q_raw;  // [BT, Hk, Dk]
  const void* k_raw;
  const void* a;      // [BT, Hv]
  const void* b;
  const float* a_log;    // [Hv]
  const float* dt_bias;  // [Hv]
  void* q;
  void* k;
  void* beta;        // [BT, Hv]
  float* log_decay;  // [BT, Hv]
};

struct NbPrologueGrad {
  const void* q_raw;
  const void* k_raw;
  const void* a;
  const void* b;
  const float* a_log;
  const float* dt_bias;
  const void* dq;   // cotangents of q, k, beta (activation dtype) and log_decay (float32)
  const void* dk;
  const void* dbeta;
  const float* dlog_decay;
  void* dq_raw;
  void* dk_raw;
  void* da;
  void* db;
  float* da_log;    // [Hv]
  float* ddt_bias;  // [Hv]
};

struct NbEpilogue {
  const void* y;  // [BT, Hv, Dv]
  const void* z;
  const float* w;  // [Dv]
  float eps;
  void* o;
};

struct NbEpilogueGrad {
  const void* y;
  const void* z;
  const float* w;
  float eps;
  const void* dout;
  void* dy;
  void* dz;
  float* dw;  // [Dv]
};

// Why the kernels cannot run p (nullptr when they can): the prologue uses Dk, the epilogue Dv; with neither flag,
// at least one of the two must be a width they take.
const char* nb_supports(const NbProblem& p, bool uses_dk, bool uses_dv);
size_t nb_workspace_bytes(const NbProblem& p);
hipError_t nb_prologue_fwd(const NbProblem& p, const NbPrologue& x, hipStream_t s);
hipError_t nb_prologue_bwd(const NbProblem& p, const NbPrologueGrad& x, void* ws, hipStream_t s);
hipError_t nb_epilogue_fwd(const NbProblem& p, const NbEpilogue& x, hipStream_t s);
hipError_t nb_epilogue_bwd(const NbProblem& p, const NbEpilogueGrad& x, void* ws, hipStream_t s);

}  // namespace qbgdn
