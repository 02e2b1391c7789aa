// Chunked design, kernel 2: the forward state pass. One block (4 waves) per (sequence, value head, 16 state rows),
// sequential over the sequence's chunks; rows of the state evolve independently (reference src/delta_grad.cpp:13),
// so a 16-row block needs no other block. Per chunk, with S the block's rows of the state at the chunk start:
//   write S to the chunk's checkpoint slot (the reference's ckpt, src/delta_grad.cpp:172-181)
//   KS = K S^T, QS = Q S^T                        [64 x 16]   wave w: positions 16w..16w+15
//   R = V - diag(exp G) KS;  Delta = T diag(beta) R
//   S <- exp(G_63) S + (diag(exp(G_63 - G)) Delta)^T K        wave w: state columns 32w..32w+31
//   Y = diag(exp G) QS + P Delta,  P = lower_incl(exp(G_i - G_j) q_i . k_j)
// All products run on v_mfma_f32_16x16x32_bf16; float32 operands (S, T diag(beta), R, Delta, P) are split into
// bf16 hi + lo pairs so the state keeps float32 accuracy, and k, q, v enter exactly (they are bf16).
#include "chunk_common.h"
#include "chunk_kernels.h"

namespace qbgdn {
namespace {

constexpr int kThreads = 256;
constexpr int kLDK = 128 + kPadB;  // bf16 row stride for Dk = 128
constexpr int kLDC = kC + kPadB;   // bf16 row stride for 64 positions

template <typename OutT>
__global__ __launch_bounds__(kThreads) void chunk_fwd_kernel(ChunkArgs a) {
  constexpr int Dk = 128;
  __shared__ __bf16 Kb[kC][kLDK], Qb[kC][kLDK];
  __shared__ __bf16 Tbh[kC][kLDC], Tbl[kC][kLDC];
  __shared__ __bf16 Sh[16][kLDK], Sl[16][kLDK];
  __shared__ __bf16 Rth[16][kLDC], Rtl[16][kLDC], Dth[16][kLDC], Dtl[16][kLDC], DDth[16][kLDC], DDtl[16][kLDC];
  __shared__ float Vs[kC][16];
  __shared__ double Gd[kC];
  __shared__ float gam[kC], Dd[kC], Bs[kC];

  const int total = a.nblk * a.Hv * a.N;
  const int wid = xcd_remap(blockIdx.x, total);
  const int blk = wid % a.nblk, hv = (wid / a.nblk) % a.Hv, n = wid / (a.nblk * a.Hv);
  const int hk = hv / (a.Hv / a.Hk), row0 = 16 * blk;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, li = lane & 15;
  const Seq sq = seq_of(a.tab, n);
  const int nch = (sq.len + kC - 1) / kC;
  OutT* y = static_cast<OutT*>(a.y);

  // State block: wave w holds rows 4g + jj, columns 32w + 16nt + li.
  f32x4 S[2];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt)
#pragma unroll
    for (int jj = 0; jj < 4; ++jj)
      S[nt][jj] = a.s0 ? a.s0[((int64_t(n) * a.Hv + hv) * a.Dv + row0 + 4 * g + jj) * Dk + 32 * w + 16 * nt + li]
                       : 0.f;

  for (int c = 0; c < nch; ++c) {
    const int64_t slot = sq.slot0 + c, tok = sq.tok0 + int64_t(c) * kC;
    const int L = min(kC, sq.len - c * kC);
    __syncthreads();  // the previous chunk's readers of LDS are done
    {
      float* ck = a.ckpt ? a.ckpt + ((slot * a.Hv + hv) * a.Dv + row0) * Dk : nullptr;
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int r = 4 * g + jj, col = 32 * w + 16 * nt + li;
          const float x = S[nt][jj];
          if (ck) ck[r * Dk + col] = x;
          const __bf16 h = (__bf16)x;
          Sh[r][col] = h;
          Sl[r][col] = (__bf16)(x - (float)h);
        }
    }
    stage_rows_bf16<Dk>(&Kb[0][0], kLDK, a.k, tok, a.Hk, hk, L, kThreads);
    stage_rows_bf16<Dk>(&Qb[0][0], kLDK, a.q, tok, a.Hk, hk, L, kThreads);
    for (int e = tid; e < kC * 16; e += kThreads) {
      const int t = e >> 4, r = e & 15;
      Vs[t][r] = t < L ? bf16_to_f32(a.v[((tok + t) * a.Hv + hv) * a.Dv + row0 + r]) : 0.f;
    }
    if (tid < kC) {
      const double* G = a.Gall + (slot * a.Hv + hv) * kC;
      const double gt = G[tid], gl = G[kC - 1];
      Gd[tid] = gt;
      gam[tid] = expf(float(gt));
      Dd[tid] = expf(float(gl - gt));
      Bs[tid] = tid < L ? bf16_to_f32(a.beta[(tok + tid) * a.Hv + hv]) : 0.f;
    }
    __syncthreads();
    {  // T diag(beta), split: thread -> row tid / 4, columns 16 (tid % 4) .. + 16
      const float* T = a.Tall + (slot * a.Hv + hv) * int64_t(kC * kC);
      const int i = tid >> 2, j0 = (tid & 3) * 16;
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const float4 t4 = *reinterpret_cast<const float4*>(T + i * kC + j0 + 4 * q4);
        const float tv[4] = {t4.x, t4.y, t4.z, t4.w};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int j = j0 + 4 * q4 + u;
          const float x = tv[u] * Bs[j];
          const __bf16 h = (__bf16)x;
          Tbh[i][j] = h;
          Tbl[i][j] = (__bf16)(x - (float)h);
        }
      }
    }
    __syncthreads();

    // KS, QS for positions 16w..: lane -> column r = li, rows i = 16w + 4g + jj.
    f32x4 ks = zero4(), qs = zero4();
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const bf16x8 ak = lds8(&Kb[16 * w + li][32 * s + 8 * g]), aq = lds8(&Qb[16 * w + li][32 * s + 8 * g]);
      const bf16x8 bh = lds8(&Sh[li][32 * s + 8 * g]), bl = lds8(&Sl[li][32 * s + 8 * g]);
      ks = mma(mma(ks, ak, bh), ak, bl);
      qs = mma(mma(qs, aq, bh), aq, bl);
    }
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int i = 16 * w + 4 * g + jj;
      const float r = Vs[i][li] - gam[i] * ks[jj];
      const __bf16 h = (__bf16)r;
      Rth[li][i] = h;
      Rtl[li][i] = (__bf16)(r - (float)h);
    }
    __syncthreads();

    // Delta = T diag(beta) R for positions 16w..
    f32x4 dl = zero4();
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const Split8 A{lds8(&Tbh[16 * w + li][32 * s + 8 * g]), lds8(&Tbl[16 * w + li][32 * s + 8 * g])};
      const Split8 B{lds8(&Rth[li][32 * s + 8 * g]), lds8(&Rtl[li][32 * s + 8 * g])};
      dl = mma3(dl, A, B);
    }
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int i = 16 * w + 4 * g + jj;
      const float x = dl[jj], xd = Dd[i] * dl[jj];
      const __bf16 h = (__bf16)x, hd = (__bf16)xd;
      Dth[li][i] = h;
      Dtl[li][i] = (__bf16)(x - (float)h);
      DDth[li][i] = hd;
      DDtl[li][i] = (__bf16)(xd - (float)hd);
    }
    __syncthreads();

    // S <- exp(G_63) S + (D Delta)^T K: wave w's columns 32w + 16nt + li, rows 4g + jj.
    const float glast = gam[kC - 1];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) S[nt][jj] *= glast;
      const int col = 32 * w + 16 * nt + li;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const Split8 A{lds8(&DDth[li][32 * s + 8 * g]), lds8(&DDtl[li][32 * s + 8 * g])};
        bf16x8 B;
#pragma unroll
        for (int j = 0; j < 8; ++j) B[j] = Kb[32 * s + 8 * g + j][col];
        S[nt] = mma2(S[nt], A, B);
      }
    }

    // Y = diag(exp G) QS + P Delta for positions i = 16w.. (P as the A operand: lane -> row i, k = j in the
    // stacked-C order of the P^T tiles below).
    f32x4 pt[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      pt[m] = zero4();
      if (m <= w) {
#pragma unroll
        for (int s = 0; s < 4; ++s)
          pt[m] = mma(pt[m], lds8(&Kb[16 * m + li][32 * s + 8 * g]), lds8(&Qb[16 * w + li][32 * s + 8 * g]));
      }
    }
    {
      const int i = 16 * w + li;
#pragma unroll
      for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int j = 16 * m + 4 * g + jj;
          pt[m][jj] = j <= i ? pt[m][jj] * expf(float(Gd[i] - Gd[j])) : 0.f;
        }
    }
    f32x4 yacc;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) yacc[jj] = gam[16 * w + 4 * g + jj] * qs[jj];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      if (32 * s <= 16 * w + 15) {
        float pv[8];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) pv[jj] = pt[2 * s][jj], pv[4 + jj] = pt[2 * s + 1][jj];
        const Split8 A = split8(pv);
        const Split8 B{lds4x2(&Dth[li][32 * s + 4 * g]), lds4x2(&Dtl[li][32 * s + 4 * g])};
        yacc = mma3(yacc, A, B);
      }
    }
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int i = 16 * w + 4 * g + jj;
      if (i < L) IO<OutT>::st(y, ((tok + i) * a.Hv + hv) * a.Dv + row0 + li, yacc[jj]);
    }
  }
  if (a.s_out) {
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj)
        a.s_out[((int64_t(n) * a.Hv + hv) * a.Dv + row0 + 4 * g + jj) * Dk + 32 * w + 16 * nt + li] = S[nt][jj];
  }
}

}  // namespace

hipError_t launch_chunk_fwd(const ChunkArgs& a, bool out_bf16, hipStream_t s) {
  const int total = a.nblk * a.Hv * a.N;
  if (out_bf16)
    hipLaunchKernelGGL(chunk_fwd_kernel<bf16_t>, dim3(total), dim3(kThreads), 0, s, a);
  else
    hipLaunchKernelGGL(chunk_fwd_kernel<float>, dim3(total), dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace qbgdn
