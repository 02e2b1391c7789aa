// Chunked design, kernel 3: the backward state pass. One block (4 waves) per (sequence, value head, 16 state rows),
// over the chunks in reverse. With dS the cotangent of the block's rows of the chunk's end state (ds_out for the
// last chunk), per chunk:
//   store dS (the gradient kernel needs it)
//   dDelta = P^T dY + D K dS^T,  D = diag(exp(G_63 - G))                 wave w: positions 16w..16w+15
//   dR = Tb^T dDelta;   dv = dR
//   dS <- exp(G_63) dS + (diag(exp G) dY)^T Q - (diag(exp G) dR)^T K      wave w: state columns 32w..32w+31
// This is the adjoint of the forward state pass; together with the gradient kernel it reproduces the reference's
// backward (src/delta_grad.cpp:14-18). dS0 is what remains after the first chunk. Tb and P come ready from the prep
// kernel; MFMA with split float32 operands as in the forward; the previous chunk's tiles (in the reverse sweep) are
// loaded into registers while the current one computes.
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
  __shared__ __bf16 dSh[16][kLDK], dSl[16][kLDK];
  __shared__ __bf16 dYth[16][kLDC], dYtl[16][kLDC];   // dY^T [r][i]
  __shared__ __bf16 GdYth[16][kLDC], GdYtl[16][kLDC]; // (diag(exp G) dY)^T
  __shared__ __bf16 dDth[16][kLDC], dDtl[16][kLDC];   // dDelta^T [r][j]
  __shared__ __bf16 GdRth[16][kLDC], GdRtl[16][kLDC]; // -(diag(exp G) dR)^T
  __shared__ float gam[kC], dec[kC];

  const int total = a.nblk * a.Hv * a.N;
  const int wid = xcd_remap(blockIdx.x, total);
  const int blk = wid % a.nblk, hv = (wid / a.nblk) % a.Hv, n = wid / (a.nblk * a.Hv);
  const int hk = hv / (a.Hv / a.Hk), row0 = 16 * blk;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, li = lane & 15;
  const Seq sq = seq_of(a.tab, n);
  const int nch = (sq.len + kC - 1) / kC;
  const OutT* dy = static_cast<const OutT*>(a.dy);
  OutT* dv = static_cast<OutT*>(a.dv);
  const int sk = a.Hk * Dk, sv = a.Hv * a.Dv;

  f32x4 dS[2];  // wave w: rows 4g + jj, columns 32w + 16nt + li
#pragma unroll
  for (int nt = 0; nt < 2; ++nt)
#pragma unroll
    for (int jj = 0; jj < 4; ++jj)
      dS[nt][jj] = a.ds_out
                       ? a.ds_out[((int64_t(n) * a.Hv + hv) * a.Dv + row0 + 4 * g + jj) * Dk + 32 * w + 16 * nt + li]
                       : 0.f;

  // Registers holding the previous chunk: k, q rows, dy, exp G, D, and the wave's A operands Tb^T rows 16w + li
  // and P^T rows 16w + li (k = 8g.., two k steps, hi and lo).
  bf16x8 fk[4], fq[4], ft[4], fp[4], ct[4], cp[4];
  float fdy[4], fgt[4], fgam = 0.f, fdec = 0.f;
  auto prefetch = [&](int c) {
    const int64_t slot = sq.slot0 + c, tok = sq.tok0 + int64_t(c) * kC;
    const int L = min(kC, sq.len - c * kC);
    const bf16_t* kb = a.k + tok * sk + hk * Dk;
    const bf16_t* qb = a.q + tok * sk + hk * Dk;
    const OutT* yb = dy + tok * sv + hv * a.Dv + row0;
    const Tile* tl = a.tiles + (slot * a.Hv + hv);
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int e = tid + kThreads * q4, t = e >> 4, c8 = (e & 15) * 8;
      if (t < L) {
        fk[q4] = gld8(kb + t * sk + c8);
        fq[q4] = gld8(qb + t * sk + c8);
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) fk[q4][j] = fq[q4][j] = (__bf16)0.f;
      }
      fdy[q4] = t < L ? IO<OutT>::ld(yb, int64_t(t) * sv + (e & 15)) : 0.f;
      fgt[q4] = tl->gam[t];
    }
    const int ar = (16 * w + li) * kC + 8 * g;
    ft[0] = gld8(tl->tbt_hi + ar), ft[1] = gld8(tl->tbt_lo + ar), ft[2] = gld8(tl->tbt_hi + ar + 32),
    ft[3] = gld8(tl->tbt_lo + ar + 32);
    fp[0] = gld8(tl->pt_hi + ar), fp[1] = gld8(tl->pt_lo + ar), fp[2] = gld8(tl->pt_hi + ar + 32),
    fp[3] = gld8(tl->pt_lo + ar + 32);
    if (tid < kC) fgam = tl->gam[tid], fdec = tl->dec[tid];
  };
  if (nch > 0) prefetch(nch - 1);

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
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int e = tid + kThreads * q4, t = e >> 4, r = e & 15, c8 = (e & 15) * 8;
      *reinterpret_cast<bf16x8*>(&Kb[t][c8]) = fk[q4];
      *reinterpret_cast<bf16x8*>(&Qb[t][c8]) = fq[q4];
      const float x = fdy[q4];
      const __bf16 h = (__bf16)x;
      dYth[r][t] = h;
      dYtl[r][t] = (__bf16)(x - (float)h);
      const float gx = fgt[q4] * x;
      const __bf16 gh = (__bf16)gx;
      GdYth[r][t] = gh;
      GdYtl[r][t] = (__bf16)(gx - (float)gh);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) ct[u] = ft[u], cp[u] = fp[u];
    if (tid < kC) gam[tid] = fgam, dec[tid] = fdec;
    __syncthreads();
    if (c > 0) prefetch(c - 1);

    // K dS^T for positions j = 16w..: lane -> column r = li, rows j = 16w + 4g + jj.
    f32x4 kds = zero4();
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const bf16x8 ak = lds8(&Kb[16 * w + li][32 * s + 8 * g]);
      kds = mma(mma(kds, ak, lds8(&dSh[li][32 * s + 8 * g])), ak, lds8(&dSl[li][32 * s + 8 * g]));
    }
    // dDelta rows j = 16w.. = D KdS + P^T dY (A = P^T rows j, k = i).
    f32x4 dd;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) dd[jj] = dec[16 * w + 4 * g + jj] * kds[jj];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      if (32 * s + 31 >= 16 * w) {
        const Split8 A{cp[2 * s], cp[2 * s + 1]};
        if constexpr (kExactDy) {
          dd = mma2(dd, A, lds8(&dYth[li][32 * s + 8 * g]));
        } else {
          dd = mma3(dd, A, Split8{lds8(&dYth[li][32 * s + 8 * g]), lds8(&dYtl[li][32 * s + 8 * g])});
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

    // dR = Tb^T dDelta for positions i = 16w.. (A = Tb^T rows i, k = j); dv = dR.
    f32x4 dr = zero4();
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      dr = mma3(dr, Split8{ct[2 * s], ct[2 * s + 1]}, Split8{lds8(&dDth[li][32 * s + 8 * g]), lds8(&dDtl[li][32 * s + 8 * g])});
    }
    OutT* dvb = dv + tok * sv + hv * a.Dv + row0 + li;
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int i = 16 * w + 4 * g + jj;
      if (i < L) IO<OutT>::st(dvb, int64_t(i) * sv, dr[jj]);
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
