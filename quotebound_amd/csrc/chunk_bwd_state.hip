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
constexpr int kLDK = 144;  // rows 0..3 of a transposing read on distinct banks
constexpr int kLDC = kC + kPadB;
constexpr int kLT = 80;  // Tb, P rows (swz placement)

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
  // Tb (hi, lo) and P (hi, lo) of the chunk, 64 x 64 each (swz placement; the blocks above the diagonal stay zero):
  // the A operands Tb^T and P^T come from their columns through the transposing read.
  __shared__ __align__(16) __bf16 TPL[4][kC * kLT];

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

  // One chunk's inputs, loaded into registers a chunk ahead (in the reverse sweep): k and q rows (thread e of
  // [0, 1024) in steps of 256 covers row e / 16, columns 8 (e % 16)), dy (row e / 16, state row e % 16) with its
  // exp G, the chunk's exp G and D, and the packed blocks of Tb and P (staged into LDS, where the transposing read
  // gives the A operands Tb^T and P^T). k, q, dy are read through buffer resources that end at the sequence's last
  // row, so rows past it read as zeros without a branch.
  struct Pre {
    uint4 k[4], q[4];
    uint4 tp[5];     // the packed Tb and P blocks: thread -> 16-byte units tid + 256 u of tb[0..1], p[0..1]
    uint32_t dy[4];  // raw bits (bf16 in the low half, or float32)
    float gam, dec;
  };
  // The loads come in three groups, issued at three points of the chunk before, so no wave stalls long on a full
  // load queue.
  auto load_kq = [&](Pre& f, int c) {
    const int64_t tok = sq.tok0 + int64_t(c) * kC;
    const uint32_t L = uint32_t(min(kC, sq.len - c * kC));
    const auto kr = buffer_rsrc(a.k + tok * sk + hk * Dk, L * sk * 2);
    const auto qr = buffer_rsrc(a.q + tok * sk + hk * Dk, L * sk * 2);
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int e = tid + kThreads * q4, t = e >> 4, c8 = (e & 15) * 8;
      f.k[q4] = buf_ld16(kr, uint32_t(t * sk + c8) * 2);
      f.q[q4] = buf_ld16(qr, uint32_t(t * sk + c8) * 2);
    }
  };
  auto load_tp = [&](Pre& f, int c) {
    const Tile* tl = a.tiles + ((sq.slot0 + c) * a.Hv + hv);
    const auto tr = buffer_rsrc(tl->tb[0], 4 * kTri * 2);  // tb[0], tb[1], p[0], p[1] are contiguous
#pragma unroll
    for (int u = 0; u < 5; ++u) f.tp[u] = buf_ld16(tr, uint32_t(tid + kThreads * u) * 16);
  };
  auto load_dy = [&](Pre& f, int c) {
    const int64_t tok = sq.tok0 + int64_t(c) * kC;
    const uint32_t L = uint32_t(min(kC, sq.len - c * kC));
    const auto yr = buffer_rsrc(dy + tok * sv + hv * a.Dv + row0, L * sv * uint32_t(sizeof(OutT)));
    const Tile* tl = a.tiles + ((sq.slot0 + c) * a.Hv + hv);
    f.gam = tl->gam[tid & (kC - 1)], f.dec = tl->dec[tid & (kC - 1)];
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int e = tid + kThreads * q4, t = e >> 4;
      const uint32_t yo = uint32_t(t * sv + (e & 15));
      if constexpr (kExactDy)
        f.dy[q4] = buf_ld2(yr, yo * 2);
      else
        f.dy[q4] = __float_as_uint(buf_ld4(yr, yo * 4));
    }
  };

  // dv of a chunk is stored during the chunk processed after it (after that chunk's inputs are staged), so no wait
  // for the staged loads ever covers these stores.
  auto store_dv = [&](int c, const f32x4& dr) {
    const int64_t tok = sq.tok0 + int64_t(c) * kC;
    const uint32_t L = uint32_t(min(kC, sq.len - c * kC));
    // Rows i >= L fall past the resource and are dropped.
    const auto vr = buffer_rsrc(dv + tok * sv + hv * a.Dv + row0, L * sv * uint32_t(sizeof(OutT)));
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) BufIO<OutT>::st(vr, uint32_t((16 * w + 4 * g + jj) * sv + li), dr[jj]);
  };

  auto step = [&](int c, Pre& f, Pre& nxt, f32x4& dr) {
    const int64_t slot = sq.slot0 + c;
    __syncthreads();
    // Stage the chunk first: the waits for its loads then come before this chunk's own stores.
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int e = tid + kThreads * q4, t = e >> 4, r = e & 15, c8 = (e & 15) * 8;
      *reinterpret_cast<uint4*>(&Kb[t][c8]) = f.k[q4];
      *reinterpret_cast<uint4*>(&Qb[t][c8]) = f.q[q4];
      const float x = kExactDy ? __uint_as_float(f.dy[q4] << 16) : __uint_as_float(f.dy[q4]);
      const __bf16 h = (__bf16)x;
      dYth[r][t] = h;
      dYtl[r][t] = (__bf16)(x - (float)h);
    }
    if (tid < kC) gam[tid] = f.gam, dec[tid] = f.dec;
    // The packed blocks to their places: unit e of a matrix half is row (e % 32) / 2, columns 8 (e % 2) .. of
    // block e / 32 = (I, J) in the order of tri_off.
#pragma unroll
    for (int u = 0; u < 5; ++u) {
      const int x = tid + kThreads * u, m = x / 320, e = x - 320 * m, b = e >> 5;
      const int I = (b >= 1) + (b >= 3) + (b >= 6), J = b - I * (I + 1) / 2;
      *reinterpret_cast<uint4*>(&TPL[m][swz(16 * I + ((e & 31) >> 1), 16 * J + 8 * (e & 1), kLT)]) = f.tp[u];
    }
    if (c + 1 < nch) store_dv(c + 1, dr);
    {
      const auto out = buffer_rsrc(a.dsend + ((slot * a.Hv + hv) * a.Dv + row0) * Dk, 16 * Dk * 4);
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int r = 4 * g + jj, col = 32 * w + 16 * nt + li;
          const float x = dS[nt][jj];
          BufIO<float>::st(out, uint32_t(r * Dk + col), x);
          const __bf16 h = (__bf16)x;
          dSh[r][col] = h;
          dSl[r][col] = (__bf16)(x - (float)h);
        }
    }
    __syncthreads();
    if (c > 0) load_kq(nxt, c - 1);
    // (diag(exp G) dY)^T, split (exp G is in LDS now); read in the state update.
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int e = tid + kThreads * q4, t = e >> 4, r = e & 15;
      const float x = kExactDy ? __uint_as_float(f.dy[q4] << 16) : __uint_as_float(f.dy[q4]);
      const float gx = gam[t] * x;
      const __bf16 gh = (__bf16)gx;
      GdYth[r][t] = gh;
      GdYtl[r][t] = (__bf16)(gx - (float)gh);
    }

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
        // P^T rows j = 16w + li, k = i: column j of P, rows 32s..
        const Split8 A{lds_tr8s(&TPL[2][32 * s * kLT + 16 * w], kLT, tid), lds_tr8s(&TPL[3][32 * s * kLT + 16 * w], kLT, tid)};
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
    if (c > 0) load_tp(nxt, c - 1);

    // dR = Tb^T dDelta for positions i = 16w.. (A = Tb^T rows i, k = j); dv = dR.
    dr = zero4();
#pragma unroll
    for (int s = 0; s < 2; ++s)
      if (32 * s + 31 >= 16 * w)  // Tb^T is zero below the diagonal
        dr = mma3(dr,
                  Split8{lds_tr8s(&TPL[0][32 * s * kLT + 16 * w], kLT, tid),
                         lds_tr8s(&TPL[1][32 * s * kLT + 16 * w], kLT, tid)},  // Tb^T rows i, k = j
                  Split8{lds8(&dDth[li][32 * s + 8 * g]), lds8(&dDtl[li][32 * s + 8 * g])});
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int i = 16 * w + 4 * g + jj;
      const float x = -gam[i] * dr[jj];
      const __bf16 h = (__bf16)x;
      GdRth[li][i] = h;
      GdRtl[li][i] = (__bf16)(x - (float)h);
    }
    __syncthreads();
    if (c > 0) load_dy(nxt, c - 1);

    // dS <- exp(G_63) dS + (diag(exp G) dY)^T Q - (diag(exp G) dR)^T K.
    const float glast = gam[kC - 1];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) dS[nt][jj] *= glast;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const bf16x8 bq = lds_tr8(&Qb[32 * s][32 * w + 16 * nt], kLDK, tid);  // rows 32s.., this lane's state column
        const bf16x8 bk = lds_tr8(&Kb[32 * s][32 * w + 16 * nt], kLDK, tid);
        dS[nt] = mma2(dS[nt], Split8{lds8(&GdYth[li][32 * s + 8 * g]), lds8(&GdYtl[li][32 * s + 8 * g])}, bq);
        dS[nt] = mma2(dS[nt], Split8{lds8(&GdRth[li][32 * s + 8 * g]), lds8(&GdRtl[li][32 * s + 8 * g])}, bk);
      }
    }
  };

  // The blocks above the diagonal of Tb and P are zero and never written by the staging.
  for (int x = tid; x < 4 * kC * kC / 8; x += kThreads) {
    const int m = x >> 9, r = (x >> 3) & 63, c = (x & 7) * 8;
    if ((c >> 4) > (r >> 4)) *reinterpret_cast<uint4*>(&TPL[m][swz(r, c, kLT)]) = uint4{0u, 0u, 0u, 0u};
  }
  // Two register sets in turn: chunk c computes from one while chunk c - 1 loads into the other.
  Pre pa, pb;
  f32x4 dr = zero4();
  if (nch > 0) load_kq(pa, nch - 1), load_tp(pa, nch - 1), load_dy(pa, nch - 1);
  for (int c = nch - 1; c >= 0; c -= 2) {
    step(c, pa, pb, dr);
    if (c > 0) step(c - 1, pb, pa, dr);
  }
  if (nch > 0) store_dv(0, dr);
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
