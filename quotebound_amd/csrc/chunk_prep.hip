// Chunked design, kernel 1 (prep), one block per (chunk slot, value head): the chunk's log-decay cumsum G (fp64,
// so G_i - G_j keeps its bits when |G| is large) and T = (I + A)^-1 with A = strict_lower(diag(beta) (E * K K^T)),
// E_ij = exp(G_i - G_j), the UT transform of the chunk's delta rule: Delta = T diag(beta) (V - diag(exp G) K S0^T)
// gives every step's delta_t = beta_t (v_t - u_t) of the recurrence (reference src/delta_grad.cpp:14) at once.
// K K^T runs on MFMA (bf16 inputs are exact, fp32 accumulation); the inverse is blocked forward substitution in
// fp32: 16 x 16 diagonal blocks by substitution, off-diagonal blocks T_IJ = -T_II sum_K A_IK T_KJ by distance.
#include "chunk_common.h"
#include "chunk_kernels.h"

namespace qbgdn {
namespace {

constexpr int kThreads = 256;
constexpr int kLDK = 128 + kPadB;
constexpr int kLDF = kC + 1;  // float rows, padded

__global__ __launch_bounds__(kThreads) void chunk_prep_kernel(ChunkArgs a) {
  __shared__ __bf16 Kb[kC][kLDK];
  __shared__ float Am[kC][kLDF];
  __shared__ float Tm[kC][kLDF];
  __shared__ float Ws[3][16][17];
  __shared__ double Gd[kC];
  __shared__ float Bs[kC];

  const int total = int(a.lay.NC) * a.Hv;
  const int wid = xcd_remap(blockIdx.x, total);
  const int64_t slot = wid / a.Hv;
  const int hv = wid % a.Hv, hk = hv / (a.Hv / a.Hk);
  const SlotPos sp = slot_pos(a.tab, slot);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, li = lane & 15;

  stage_rows_bf16<128>(&Kb[0][0], kLDK, a.k, sp.tok, a.Hk, hk, sp.L, kThreads);
  if (tid < kC) {
    const int t = tid;
    Gd[t] = t < sp.L ? log_decay(a.g, (sp.tok + t) * a.Hv + hv, a.g_is_log) : 0.0;
    Bs[t] = t < sp.L ? bf16_to_f32(a.beta[(sp.tok + t) * a.Hv + hv]) : 0.f;
  }
  // Inclusive prefix sum of the log-decays (Hillis-Steele, fp64).
  for (int off = 1; off < kC; off <<= 1) {
    __syncthreads();
    const double add = (tid < kC && tid >= off) ? Gd[tid - off] : 0.0;
    __syncthreads();
    if (tid < kC) Gd[tid] += add;
  }
  __syncthreads();

  // A = strict_lower(beta_i exp(G_i - G_j) k_i . k_j); wave w computes row strip w.
  for (int nj = 0; nj <= w; ++nj) {
    f32x4 acc = zero4();
#pragma unroll
    for (int s = 0; s < 4; ++s)
      acc = mma(acc, lds8(&Kb[16 * w + li][32 * s + 8 * g]), lds8(&Kb[16 * nj + li][32 * s + 8 * g]));
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int i = 16 * w + 4 * g + jj, j = 16 * nj + li;
      Am[i][j] = j < i ? Bs[i] * expf(float(Gd[i] - Gd[j])) * acc[jj] : 0.f;
    }
  }
  __syncthreads();

  // Diagonal blocks: column j of block bd by forward substitution (one thread per column).
  if (tid < kC) {
    const int bd = tid >> 4, jl = tid & 15, j = 16 * bd + jl;
    for (int il = 0; il < 16; ++il) {
      const int i = 16 * bd + il;
      float x = il == jl ? 1.f : 0.f;
      if (il > jl) {
        for (int k = j; k < i; ++k) x -= Am[i][k] * Tm[k][j];
      }
      Tm[i][j] = x;
    }
  }
  // Blocks above the diagonal are zero.
  for (int e = tid; e < kC * kC; e += kThreads) {
    const int i = e / kC, j = e % kC;
    if ((j >> 4) > (i >> 4)) Tm[i][j] = 0.f;
  }
  __syncthreads();
  // Off-diagonal blocks at distance d = I - J: W = sum_{J <= K < I} A_IK T_KJ, then T_IJ = -T_II W.
  for (int d = 1; d < 4; ++d) {
    const int nblk = 4 - d;
    for (int e = tid; e < nblk * 256; e += kThreads) {
      const int b = e >> 8, I = d + b, J = I - d, il = (e & 255) >> 4, jl = e & 15;
      const int i = 16 * I + il, j = 16 * J + jl;
      float acc = 0.f;
      for (int k = 16 * J; k < 16 * I; ++k) acc += Am[i][k] * Tm[k][j];
      Ws[b][il][jl] = acc;
    }
    __syncthreads();
    for (int e = tid; e < nblk * 256; e += kThreads) {
      const int b = e >> 8, I = d + b, J = I - d, il = (e & 255) >> 4, jl = e & 15;
      float acc = 0.f;
      for (int m = 0; m <= il; ++m) acc += Tm[16 * I + il][16 * I + m] * Ws[b][m][jl];
      Tm[16 * I + il][16 * J + jl] = -acc;
    }
    __syncthreads();
  }

  float* Tout = a.Tall + (slot * a.Hv + hv) * int64_t(kC * kC);
  for (int e = tid; e < kC * kC; e += kThreads) Tout[e] = Tm[e / kC][e % kC];
  if (tid < kC) a.Gall[(slot * a.Hv + hv) * kC + tid] = Gd[tid];
}

}  // namespace

hipError_t launch_chunk_prep(const ChunkArgs& a, hipStream_t s) {
  const int total = int(a.lay.NC) * a.Hv;
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL(chunk_prep_kernel, dim3(total), dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace qbgdn
