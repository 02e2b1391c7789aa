// Chunked design, kernel 3: the backward state pass. One block (4 waves) per (sequence, value head, 16 state rows),
// over the chunks in reverse. With dS the cotangent of the block's rows of the chunk's end state (ds_out for the
// last chunk), per chunk:
//   store dS (the gradient kernel needs it)
//   dDelta = P^T dY + D K dS^T,  D = diag(exp(G_63 - G))                 wave w: positions 16w..16w+15
//   dR = (T diag(beta))^T dDelta;   dv = dR
//   dS <- exp(G_63) dS + (diag(exp G) dY)^T Q - (diag(exp G) dR)^T K      wave w: state columns 32w..32w+31
// This is the adjoint of the forward state pass; together with the gradient kernel it reproduces the reference's
// backward (src/delta_grad.cpp:14-18). dS0 is what remains after the first chunk. MFMA with split float32 operands
// as in the forward.
#include <type_traits>

#include "chunk_common.h"
#include "chunk_kernels.h"

namespace qbgdn {
namespace {

constexpr int kThreads = 256;
constexpr int kLDK = 128 + kPadB;
constexpr int kLDC = kC + kPadB;

template <typename OutT>
__global__ __launch_bounds__(kThreads) void chunk_bwd_state_kernel(ChunkArgs a) {
  constexpr int Dk = 128;
  constexpr bool kExactDy = std::is_same<OutT, bf16_t>::value;  // bf16 cotangents enter MFMA exactly
  __shared__ __bf16 Kb[kC][kLDK], Qb[kC][kLDK];
  __shared__ __bf16 Tbth[kC][kLDC], Tbtl[kC][kLDC];  // (T diag(beta))^T, row i, column j
  __shared__ __bf16 dSh[16][kLDK], dSl[16][kLDK];
  __shared__ __bf16 dYth[16][kLDC], dYtl[16][kLDC];   // dY^T [r][i]
  __shared__ __bf16 GdYth[16][kLDC], GdYtl[16][kLDC]; // (diag(exp G) dY)^T
  __shared__ __bf16 dDth[16][kLDC], dDtl[16][kLDC];   // dDelta^T [r][j]
  __shared__ __bf16 GdRth[16][kLDC], GdRtl[16][kLDC]; // -(diag(exp G) dR)^T
  __shared__ double Gd[kC];
  __shared__ float gam[kC], Dd[kC], Bs[kC];

  const int total = a.nblk * a.Hv * a.N;
  const int wid = xcd_remap(blockIdx.x, total);
  const int blk = wid % a.nblk, hv = (wid / a.nblk) % a.Hv, n = wid / (a.nblk * a.Hv);
  const int hk = hv / (a.Hv / a.Hk), row0 = 16 * blk;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, li = lane & 15;
  const Seq sq = seq_of(a.tab, n);
  const int nch = (sq.len + kC - 1) / kC;
  const OutT* dy = static_cast<const OutT*>(a.dy);
  OutT* dv = static_cast<OutT*>(a.dv);

  f32x4 dS[2];  // wave w: rows 4g + jj, columns 32w + 16nt + li
#pragma unroll
  for (int nt = 0; nt < 2; ++nt)
#pragma unroll
    for (int jj = 0; jj < 4; ++jj)
      dS[nt][jj] = a.ds_out
                       ? a.ds_out[((int64_t(n) * a.Hv + hv) * a.Dv + row0 + 4 * g + jj) * Dk + 32 * w + 16 * nt + li]
                       : 0.f;

  for (int c = nch - 1; c >= 0; --c) {
    const int64_t slot = sq.slot0 + c, tok = sq.tok0 + int64_t(c) * kC;
    const int L = min(kC, sq.len - c * kC);
    __syncthreads();
    {
      float* out = a.dsend + ((slot * a.Hv + hv) * a.Dv + row0) * Dk;
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int r = 4 * g + jj, col = 32 * w + 16 * nt + li;
          const float x = dS[nt][jj];
          out[r * Dk + col] = x;
          const __bf16 h = (__bf16)x;
          dSh[r][col] = h;
          dSl[r][col] = (__bf16)(x - (float)h);
        }
    }
    stage_rows_bf16<Dk>(&Kb[0][0], kLDK, a.k, tok, a.Hk, hk, L, kThreads);
    stage_rows_bf16<Dk>(&Qb[0][0], kLDK, a.q, tok, a.Hk, hk, L, kThreads);
    if (tid < kC) {
      const double* G = a.Gall + (slot * a.Hv + hv) * kC;
      const double gt = G[tid], gl = G[kC - 1];
      Gd[tid] = gt;
      gam[tid] = expf(float(gt));
      Dd[tid] = expf(float(gl - gt));
      Bs[tid] = tid < L ? bf16_to_f32(a.beta[(tok + tid) * a.Hv + hv]) : 0.f;
    }
    __syncthreads();
    for (int e = tid; e < kC * 16; e += kThreads) {
      const int t = e >> 4, r = e & 15;
      const float x = t < L ? IO<OutT>::ld(dy, ((tok + t) * a.Hv + hv) * a.Dv + row0 + r) : 0.f;
      const __bf16 h = (__bf16)x;
      dYth[r][t] = h;
      dYtl[r][t] = (__bf16)(x - (float)h);
      const float gx = gam[t] * x;
      const __bf16 gh = (__bf16)gx;
      GdYth[r][t] = gh;
      GdYtl[r][t] = (__bf16)(gx - (float)gh);
    }
    {  // (T diag(beta))^T: Tbt[i][j] = T[j][i] beta_i; thread -> row j = tid / 4 of T, columns 16 (tid % 4) ..
      const float* T = a.Tall + (slot * a.Hv + hv) * int64_t(kC * kC);
      const int j = tid >> 2, i0 = (tid & 3) * 16;
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const float4 t4 = *reinterpret_cast<const float4*>(T + j * kC + i0 + 4 * q4);
        const float tv[4] = {t4.x, t4.y, t4.z, t4.w};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int i = i0 + 4 * q4 + u;
          const float x = tv[u] * Bs[i];
          const __bf16 h = (__bf16)x;
          Tbth[i][j] = h;
          Tbtl[i][j] = (__bf16)(x - (float)h);
        }
      }
    }
    __syncthreads();

    // K dS^T for positions j = 16w..: lane -> column r = li, rows j = 16w + 4g + jj.
    f32x4 kds = zero4();
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const bf16x8 ak = lds8(&Kb[16 * w + li][32 * s + 8 * g]);
      kds = mma(mma(kds, ak, lds8(&dSh[li][32 * s + 8 * g])), ak, lds8(&dSl[li][32 * s + 8 * g]));
    }
    // P^T rows j = 16w + li (k = i): tiles of P = Q K^T with lane -> column j, rows i = 16m + 4g + jj.
    f32x4 pq[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      pq[m] = zero4();
      if (m >= w) {
#pragma unroll
        for (int s = 0; s < 4; ++s)
          pq[m] = mma(pq[m], lds8(&Qb[16 * m + li][32 * s + 8 * g]), lds8(&Kb[16 * w + li][32 * s + 8 * g]));
        const int j = 16 * w + li;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int i = 16 * m + 4 * g + jj;
          pq[m][jj] = i >= j ? pq[m][jj] * expf(float(Gd[i] - Gd[j])) : 0.f;
        }
      }
    }
    f32x4 dd;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) dd[jj] = Dd[16 * w + 4 * g + jj] * kds[jj];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      if (2 * s + 1 >= w) {
        float pv[8];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) pv[jj] = pq[2 * s][jj], pv[4 + jj] = pq[2 * s + 1][jj];
        const Split8 A = split8(pv);
        if constexpr (kExactDy) {
          dd = mma2(dd, A, lds4x2(&dYth[li][32 * s + 4 * g]));
        } else {
          dd = mma3(dd, A, Split8{lds4x2(&dYth[li][32 * s + 4 * g]), lds4x2(&dYtl[li][32 * s + 4 * g])});
        }
      }
    }
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int j = 16 * w + 4 * g + jj;
      const __bf16 h = (__bf16)dd[jj];
      dDth[li][j] = h;
      dDtl[li][j] = (__bf16)(dd[jj] - (float)h);
    }
    __syncthreads();

    // dR = (T diag(beta))^T dDelta for positions i = 16w..; dv = dR.
    f32x4 dr = zero4();
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const Split8 A{lds8(&Tbth[16 * w + li][32 * s + 8 * g]), lds8(&Tbtl[16 * w + li][32 * s + 8 * g])};
      const Split8 B{lds8(&dDth[li][32 * s + 8 * g]), lds8(&dDtl[li][32 * s + 8 * g])};
      dr = mma3(dr, A, B);
    }
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int i = 16 * w + 4 * g + jj;
      if (i < L) IO<OutT>::st(dv, ((tok + i) * a.Hv + hv) * a.Dv + row0 + li, dr[jj]);
      const float x = -gam[i] * dr[jj];
      const __bf16 h = (__bf16)x;
      GdRth[li][i] = h;
      GdRtl[li][i] = (__bf16)(x - (float)h);
    }
    __syncthreads();

    // dS <- exp(G_63) dS + (diag(exp G) dY)^T Q - (diag(exp G) dR)^T K.
    const float glast = gam[kC - 1];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) dS[nt][jj] *= glast;
      const int col = 32 * w + 16 * nt + li;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        bf16x8 bq, bk;
#pragma unroll
        for (int j = 0; j < 8; ++j) bq[j] = Qb[32 * s + 8 * g + j][col], bk[j] = Kb[32 * s + 8 * g + j][col];
        dS[nt] = mma2(dS[nt], Split8{lds8(&GdYth[li][32 * s + 8 * g]), lds8(&GdYtl[li][32 * s + 8 * g])}, bq);
        dS[nt] = mma2(dS[nt], Split8{lds8(&GdRth[li][32 * s + 8 * g]), lds8(&GdRtl[li][32 * s + 8 * g])}, bk);
      }
    }
  }
  if (a.ds0) {
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj)
        a.ds0[((int64_t(n) * a.Hv + hv) * a.Dv + row0 + 4 * g + jj) * Dk + 32 * w + 16 * nt + li] = dS[nt][jj];
  }
}

}  // namespace

hipError_t launch_chunk_bwd_state(const ChunkArgs& a, bool out_bf16, hipStream_t s) {
  const int total = a.nblk * a.Hv * a.N;
  if (out_bf16)
    hipLaunchKernelGGL(chunk_bwd_state_kernel<bf16_t>, dim3(total), dim3(kThreads), 0, s, a);
  else
    hipLaunchKernelGGL(chunk_bwd_state_kernel<float>, dim3(total), dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace qbgdn
