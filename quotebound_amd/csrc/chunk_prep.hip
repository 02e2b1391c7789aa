// Chunked design, kernel 1 (prep), one block per (chunk slot, value head): everything about the chunk that does not
// depend on the state, written once as MFMA-ready operands (the Tile record, chunk_common.h).
//   G = cumsum of the log-decays (fp64, so G_i - G_j keeps its bits when |G| is large)
//   A = strict_lower(diag(beta) (E * K K^T)),  T = (I + A)^-1,  Tb = T diag(beta)
//   P = lower_incl(E * Q K^T),  E_ij = exp(G_i - G_j)
// T is the UT transform of the chunk's delta rule: Delta = Tb (V - diag(exp G) K S0^T) gives every step's
// delta_t = beta_t (v_t - u_t) of the recurrence (reference src/delta_grad.cpp:14) at once. K K^T and Q K^T run on
// MFMA (bf16 inputs are exact, fp32 accumulation); the inverse is blocked forward substitution in fp32: each 16 x 16
// diagonal block by substitution with the column held in registers, then T_IJ = -T_II sum_K A_IK T_KJ by distance.
#include "chunk_common.h"
#include "chunk_kernels.h"

namespace qbgdn {
namespace {

constexpr int kThreads = 256;
constexpr int kLDK = 128 + kPadB;
constexpr int kLDF = kC + 1;  // float rows, padded

__global__ __launch_bounds__(kThreads) void chunk_prep_kernel(ChunkArgs a) {
  __shared__ __bf16 Kb[kC][kLDK], Qb[kC][kLDK];
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
  Tile* tile = a.tiles + (slot * a.Hv + hv);

  stage_rows_bf16<128>(&Kb[0][0], kLDK, a.k, sp.tok, a.Hk, hk, sp.L, kThreads);
  stage_rows_bf16<128>(&Qb[0][0], kLDK, a.q, sp.tok, a.Hk, hk, sp.L, kThreads);
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
  if (tid < kC) {
    const double G = Gd[tid];
    tile->beta[tid] = Bs[tid];
    tile->gam[tid] = expf(float(G));
    tile->dec[tid] = expf(float(Gd[kC - 1] - G));
    tile->G[tid] = float(G);
  }

  // Row strip w: A (into LDS) and P (straight out), lane -> column j = 16 nj + li, rows i = 16 w + 4 g + jj.
  for (int nj = 0; nj < 4; ++nj) {
    f32x4 kk = zero4(), qk = zero4();
    if (nj <= w) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const bf16x8 b = lds8(&Kb[16 * nj + li][32 * s + 8 * g]);
        kk = mma(kk, lds8(&Kb[16 * w + li][32 * s + 8 * g]), b);
        qk = mma(qk, lds8(&Qb[16 * w + li][32 * s + 8 * g]), b);
      }
    }
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int i = 16 * w + 4 * g + jj, j = 16 * nj + li;
      const float e = j <= i ? expf(float(Gd[i] - Gd[j])) : 0.f;
      Am[i][j] = j < i ? Bs[i] * e * kk[jj] : 0.f;
      const float p = e * qk[jj];
      const bf16_t h = __builtin_bit_cast(bf16_t, (__bf16)p);
      const bf16_t l = __builtin_bit_cast(bf16_t, (__bf16)(p - bf16_to_f32(h)));
      tile->p_hi[i * kC + j] = h, tile->p_lo[i * kC + j] = l;
      tile->pt_hi[j * kC + i] = h, tile->pt_lo[j * kC + i] = l;
    }
  }
  __syncthreads();

  // Diagonal blocks: thread -> column j of block bd; the column lives in registers through the substitution.
  if (tid < kC) {
    const int bd = tid >> 4, jl = tid & 15, b0 = 16 * bd;
    float x[16];
#pragma unroll
    for (int il = 0; il < 16; ++il) {
      float v = il == jl ? 1.f : 0.f;
#pragma unroll
      for (int kl = 0; kl < il; ++kl) v -= kl >= jl ? Am[b0 + il][b0 + kl] * x[kl] : 0.f;
      x[il] = il >= jl ? v : 0.f;
    }
#pragma unroll
    for (int il = 0; il < 16; ++il) Tm[b0 + il][b0 + jl] = x[il];
  }
  for (int e = tid; e < kC * kC; e += kThreads) {  // blocks above the diagonal are zero
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

  // T, Tb = T diag(beta) and Tb^T: thread -> row tid / 4, columns 16 (tid % 4) .. (of T for T and Tb; of Tb^T,
  // i.e. column tid / 4 of Tb, for Tb^T).
  {
    const int i = tid >> 2, j0 = (tid & 3) * 16;
    bf16x8 h[2], l[2], th[2], tl[2];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const float t = Tm[i][j0 + u], x = t * Bs[j0 + u], xt = Tm[j0 + u][i] * Bs[i];
      tile->t[i * kC + j0 + u] = t;
      const __bf16 hh = (__bf16)x, ht = (__bf16)xt;
      h[u >> 3][u & 7] = hh;
      l[u >> 3][u & 7] = (__bf16)(x - (float)hh);
      th[u >> 3][u & 7] = ht;
      tl[u >> 3][u & 7] = (__bf16)(xt - (float)ht);
    }
    *reinterpret_cast<bf16x8*>(&tile->tb_hi[i * kC + j0]) = h[0];
    *reinterpret_cast<bf16x8*>(&tile->tb_hi[i * kC + j0 + 8]) = h[1];
    *reinterpret_cast<bf16x8*>(&tile->tb_lo[i * kC + j0]) = l[0];
    *reinterpret_cast<bf16x8*>(&tile->tb_lo[i * kC + j0 + 8]) = l[1];
    *reinterpret_cast<bf16x8*>(&tile->tbt_hi[i * kC + j0]) = th[0];
    *reinterpret_cast<bf16x8*>(&tile->tbt_hi[i * kC + j0 + 8]) = th[1];
    *reinterpret_cast<bf16x8*>(&tile->tbt_lo[i * kC + j0]) = tl[0];
    *reinterpret_cast<bf16x8*>(&tile->tbt_lo[i * kC + j0 + 8]) = tl[1];
  }
}

}  // namespace

hipError_t launch_chunk_prep(const ChunkArgs& a, hipStream_t s) {
  const int total = int(a.lay.NC) * a.Hv;
  if (total == 0) return hipSuccess;
  hipLaunchKernelGGL(chunk_prep_kernel, dim3(total), dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace qbgdn
