// The arithmetic of the layer's prologue (reference src/deltanet.cpp:22-33, 94-100), shared by the separate pass
// (neighbours.hip) and the chunked design's fused forward and backward (chunk_prep.hip, chunk_bwd_grads.hip), so
// that both form the same bits: q = s_q rms_norm(q_raw), k = s_k rms_norm(k_raw) (no weight, eps 1e-6), beta =
// sigmoid(b), log-decay = -exp(A_log) softplus(a + dt_bias), each output rounded to the activation dtype where the
// reference's op rounds it, arithmetic float32.
#pragma once
#include "gdn_common.h"

namespace qbgdn {

constexpr float kNormEps = 1e-6f;  // the q/k rms_norm's eps (src/deltanet.cpp:96-97)

template <typename T>
__device__ __forceinline__ float rnd(float x) {  // the activation dtype's rounding
  if constexpr (sizeof(T) == 2) return float(static_cast<__bf16>(x));
  return x;
}

// The hardware exp2 and reciprocal (a few float32 ulps).
__device__ __forceinline__ float sigmoidf(float x) { return __builtin_amdgcn_rcpf(1.f + __expf(-x)); }
__device__ __forceinline__ float rsqrt_mean(float ss, int n, float eps) { return __builtin_amdgcn_rsqf(ss / n + eps); }
__device__ __forceinline__ float softplusf(float x) { return fmaxf(x, 0.f) + log1pf(expf(-fabsf(x))); }

// The sum of squares a lane contributes from its 8 consecutive elements of a row, in order.
__device__ __forceinline__ float sumsq8(const float (&x)[8]) {
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) ss += x[e] * x[e];
  return ss;
}

// One lane's 8 elements of a normalised q or k row: x <- rnd(s rnd(x rho)), rho = (mean(x^2) + eps)^-1/2 over the
// D elements of the row, ss_row being the row's sum of squares (the lane sums of sumsq8, reduced over the row's
// lanes).
template <typename T>
__device__ __forceinline__ void norm_row8(float (&x)[8], float ss_row, int D, float s) {
  const float rho = rsqrt_mean(ss_row, D, kNormEps);
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = rnd<T>(s * rnd<T>(x[e] * rho));
}

// The q/k normalisation's backward for one lane's 8 elements of a row: g holds the cotangent of the normalised row
// (dout) and gets s dout; the lane sums of sum(x^2) and sum(g x) come back, to be reduced over the row's lanes and
// handed to norm_bwd_apply, which leaves dx = rho g - rho^3 x sum(g x) / D in x.
__device__ __forceinline__ void norm_bwd_sums(const float (&x)[8], float (&g)[8], float s, float& ss, float& gx) {
  ss = 0.f, gx = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    g[e] *= s;
    ss += x[e] * x[e];
    gx += g[e] * x[e];
  }
}
__device__ __forceinline__ void norm_bwd_apply(float (&x)[8], const float (&g)[8], float ss_row, float gx_row, int D) {
  const float rho = rsqrt_mean(ss_row, D, kNormEps);
  const float c = rho * rho * rho * gx_row / D;
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = rho * g[e] - c * x[e];
}

// The gates' backward for one (token, value head): db from the cotangent of beta (already in the activation dtype),
// da from that of the log-decay, and the terms of dA_log (dlog_decay * log_decay) and ddt_bias (da unrounded).
template <typename T>
__device__ __forceinline__ void gate_bwd(float a, float b, float dbeta, float dlog, float ea, float dt_bias,
                                         float& da, float& db, float& pa, float& pd) {
  const float sb = sigmoidf(b);
  db = dbeta * sb * (1.f - sb);
  const float x = rnd<T>(a + dt_bias);
  da = -dlog * ea * sigmoidf(x);
  pa = dlog * (-ea * rnd<T>(softplusf(x)));
  pd = da;
}

// beta and the log-decay of one (token, value head) from b and a.
template <typename T>
__device__ __forceinline__ float gate_beta(float b) { return rnd<T>(sigmoidf(b)); }
template <typename T>
__device__ __forceinline__ float gate_log_decay(float a, float a_log, float dt_bias) {
  return -expf(a_log) * rnd<T>(softplusf(rnd<T>(a + dt_bias)));
}

}  // namespace qbgdn
