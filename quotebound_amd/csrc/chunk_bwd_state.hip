// Chunked design, kernel 3: the backward state pass. One block (8 waves) per (sequence, value head, 16 state rows),
// over the chunks in reverse. With dS the cotangent of the block's rows of the chunk's end state (ds_out for the
// last chunk), per chunk:
//   store dS (the gradient kernel needs it)
//   dDelta = P^T dY + D K dS^T,  D = diag(exp(G_63 - G))        waves 0-3, positions 16w..16w+15: the chain
//   dR = Tb^T dDelta;   dv = dR                                   waves 0-3
//   X = (diag(exp G) dY)^T Q                                      waves 4-7, beside the chain (no dS in it)
//   dS <- exp(G_63) dS + X - (diag(exp G) dR)^T K                 every wave: state columns 16w..16w+15
// This is the adjoint of the forward state pass; together with the gradient kernel it reproduces the reference's
// backward (src/delta_grad.cpp:14-18). dS0 is what remains after the first chunk. Tb and P come ready from the prep
// kernel; MFMA with split float32 operands as in the forward. Waves 4-7 also load and stage every chunk input, so
// the chain waves issue no loads.
#include <type_traits>

#include "chunk_common.h"
#include "chunk_kernels.h"

namespace qbgdn {
namespace {

constexpr int kThreads = 512;
// Row pitches (elements) of the swz-placed LDS matrices: 16 x an odd number.
constexpr int kLDK = 144;  // k, q rows [64][128]
constexpr int kLT = 80;    // [.][64]: Tb, P, dDelta^T, (diag(exp G) dR)^T
constexpr int kLR = 48;    // [.][16]: dS^T, dY, diag(exp G) dY (state rows as columns)
constexpr int kLX = 128 + 4;  // float32 X rows

template <typename OutT>
__global__ __launch_bounds__(kThreads) void chunk_bwd_state_kernel(ChunkArgs a) {
  constexpr int Dk = 128;
  constexpr bool kExactDy = std::is_same<OutT, bf16_t>::value;  // bf16 cotangents enter MFMA exactly
  // Every matrix is placed by swz and stored once, hi and lo: row reads and transposing reads both come free of
  // bank conflicts.
  __shared__ __align__(16) __bf16 Kb[kC * kLDK], Qb[kC * kLDK];
  __shared__ __align__(16) __bf16 dSt[2][Dk * kLR];  // dS^T [c][r]
  __shared__ __align__(16) __bf16 dYm[2][kC * kLR];  // dY [i][r]
  __shared__ __align__(16) __bf16 GdYm[2][kC * kLR]; // diag(exp G) dY [i][r]
  __shared__ __align__(16) __bf16 dDt[2][16 * kLT];  // dDelta^T [r][j]
  __shared__ __align__(16) __bf16 GdRt[2][16 * kLT]; // -(diag(exp G) dR)^T [r][i]
  __shared__ __align__(16) float Xs[16 * kLX];       // X [r][c]
  __shared__ float gam[kC], dec[kC];
  // Tb (hi, lo) and P (hi, lo) of the chunk, 64 x 64 each (swz placement; the blocks above the diagonal stay zero):
  // the A operands Tb^T and P^T come from their columns through the transposing read.
  __shared__ __align__(16) __bf16 TPL[4][kC * kLT];

  const int total = a.nblk * a.Hv * a.N;
  const int wid = xcd_remap(blockIdx.x, total);
  const int blk = wid % a.nblk, hv = (wid / a.nblk) % a.Hv, n = wid / (a.nblk * a.Hv);
  const int hk = hv / (a.Hv / a.Hk), row0 = 16 * blk;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, li = lane & 15;
  const bool side = w >= 4;
  const int wp = w & 3, u = tid & 255;  // position tile (waves 0-3); thread index within the wave group
  const Seq sq = seq_of(a.tab, n);
  const int nch = (sq.len + kC - 1) / kC;
  const OutT* dy = static_cast<const OutT*>(a.dy);
  OutT* dv = static_cast<OutT*>(a.dv);
  const int sk = a.Hk * Dk, sv = a.Hv * a.Dv;

  f32x4 dS;  // wave w: rows 4g + jj, columns 16w + li
#pragma unroll
  for (int jj = 0; jj < 4; ++jj)
    dS[jj] = a.ds_out ? a.ds_out[((int64_t(n) * a.Hv + hv) * a.Dv + row0 + 4 * g + jj) * Dk + 16 * w + li] : 0.f;

  // One chunk's inputs, loaded by waves 4-7 into registers a chunk ahead (in the reverse sweep), in two groups at
  // two barriers: k and q rows (e = u + 256 q4 covers row e / 16, columns 8 (e % 16)); then the packed blocks of Tb
  // and P (16-byte units u + 256 t of tb[0..1], p[0..1]), dy row u / 4 at state rows 4 (u % 4) .. + 3, and exp G, D
  // of position u % 64. k, q, dy are read through buffer resources that end at the sequence's last row, so rows
  // past it read as zeros without a branch.
  struct Pre {
    uint4 k[4], q[4];
    uint4 tp[5];
    uint4 dy;  // raw bits (4 bf16 in .x, .y, or 4 float32)
    float gam, dec;
  };
  auto load_kq = [&](Pre& f, int c) {
    const int64_t tok = sq.tok0 + int64_t(c) * kC;
    const uint32_t L = uint32_t(min(kC, sq.len - c * kC));
    const auto kr = buffer_rsrc(a.k + tok * sk + hk * Dk, L * sk * 2);
    const auto qr = buffer_rsrc(a.q + tok * sk + hk * Dk, L * sk * 2);
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int e = u + 256 * q4, t = e >> 4, c8 = (e & 15) * 8;
      f.k[q4] = buf_ld16(kr, uint32_t(t * sk + c8) * 2);
      f.q[q4] = buf_ld16(qr, uint32_t(t * sk + c8) * 2);
    }
  };
  auto load_rest = [&](Pre& f, int c) {
    const int64_t tok = sq.tok0 + int64_t(c) * kC;
    const uint32_t L = uint32_t(min(kC, sq.len - c * kC));
    const Tile* tl = a.tiles + ((sq.slot0 + c) * a.Hv + hv);
    const auto tr = buffer_rsrc(tl->tb[0], 4 * kTri * 2);  // tb[0], tb[1], p[0], p[1] are contiguous
#pragma unroll
    for (int t5 = 0; t5 < 5; ++t5) f.tp[t5] = buf_ld16(tr, uint32_t(u + 256 * t5) * 16);
    const auto yr = buffer_rsrc(dy + tok * sv + hv * a.Dv + row0, L * sv * uint32_t(sizeof(OutT)));
    const uint32_t yo = uint32_t((u >> 2) * sv + 4 * (u & 3));
    if constexpr (kExactDy) {
      const auto t2 = __builtin_amdgcn_raw_buffer_load_b64(yr, int(yo * 2), 0, 0);
      f.dy = uint4{t2[0], t2[1], 0u, 0u};
    } else {
      f.dy = buf_ld16(yr, yo * 4);
    }
    f.gam = tl->gam[u & (kC - 1)], f.dec = tl->dec[u & (kC - 1)];
  };

  // dv of a chunk (waves 0-3) is stored during the chunk processed after it.
  auto store_dv = [&](int c, const f32x4& dr) {
    const int64_t tok = sq.tok0 + int64_t(c) * kC;
    const uint32_t L = uint32_t(min(kC, sq.len - c * kC));
    // Rows i >= L fall past the resource and are dropped.
    const auto vr = buffer_rsrc(dv + tok * sv + hv * a.Dv + row0, L * sv * uint32_t(sizeof(OutT)));
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) BufIO<OutT>::st(vr, uint32_t((16 * wp + 4 * g + jj) * sv + li), dr[jj]);
  };

  auto step = [&](int c, Pre& f, Pre& nxt, f32x4& dr) {
    const int64_t slot = sq.slot0 + c;
    __syncthreads();
    if (side) {
      // Stage the chunk. dy's four values of row u / 4 as floats, and the same times exp G of that row (lane u / 4
      // of this wave holds it: every wave of the group loads exp G of position lane).
      const int yt = u >> 2, yr4 = 4 * (u & 3);
      float yv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t b = kExactDy ? (j & 1 ? (&f.dy.x)[j >> 1] & 0xffff0000u : (&f.dy.x)[j >> 1] << 16) : (&f.dy.x)[j];
        yv[j] = __uint_as_float(b);
      }
      const float gy = __shfl(f.gam, yt);
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int e = u + 256 * q4, t = e >> 4, c8 = (e & 15) * 8;
        *reinterpret_cast<uint4*>(&Kb[swz(t, c8, kLDK)]) = f.k[q4];
        *reinterpret_cast<uint4*>(&Qb[swz(t, c8, kLDK)]) = f.q[q4];
      }
      put4(dYm[0], dYm[1], swz(yt, yr4, kLR), yv[0], yv[1], yv[2], yv[3]);
      put4(GdYm[0], GdYm[1], swz(yt, yr4, kLR), gy * yv[0], gy * yv[1], gy * yv[2], gy * yv[3]);
      if (u < kC) gam[u] = f.gam, dec[u] = f.dec;
      // The packed blocks to their places: unit e of a matrix half is row (e % 32) / 2, columns 8 (e % 2) .. of
      // block e / 32 = (I, J) in the order of tri_off.
#pragma unroll
      for (int t5 = 0; t5 < 5; ++t5) {
        const int x = u + 256 * t5, m = x / 320, e = x - 320 * m, b = e >> 5;
        const int I = (b >= 1) + (b >= 3) + (b >= 6), J = b - I * (I + 1) / 2;
        *reinterpret_cast<uint4*>(&TPL[m][swz(16 * I + ((e & 31) >> 1), 16 * J + 8 * (e & 1), kLT)]) = f.tp[t5];
      }
    } else if (c + 1 < nch) {
      store_dv(c + 1, dr);
    }
    {  // dS to the workspace and, as dS^T (four consecutive state rows per lane), to LDS.
      const auto out = buffer_rsrc(a.dsend + ((slot * a.Hv + hv) * a.Dv + row0) * Dk, 16 * Dk * 4);
      const int col = 16 * w + li;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) BufIO<float>::st(out, uint32_t((4 * g + jj) * Dk + col), dS[jj]);
      put4(dSt[0], dSt[1], swz(col, 4 * g, kLR), dS);
    }
    __syncthreads();

    if (!side) {
      // K dS^T for positions j = 16wp..: lane -> column r = li, rows j = 16wp + 4g + jj. B = dS rows r, k = c,
      // through the transposing read of dS^T.
      f32x4 kds = zero4();
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const bf16x8 ak = lds8(&Kb[swz(16 * wp + li, 32 * s + 8 * g, kLDK)]);
        kds = mma(mma(kds, ak, lds_tr8s(dSt[0] + 32 * s * kLR, kLR, tid)), ak, lds_tr8s(dSt[1] + 32 * s * kLR, kLR, tid));
      }
      // dDelta rows j = 16wp.. = D KdS + P^T dY (A = P^T rows j, k = i; B = dY rows i through the transposing
      // read). Both k steps for every wave: the ones above the diagonal add zeros, and the waves that need both
      // set the pace, so skipping them would only add branches.
      f32x4 dd;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) dd[jj] = dec[16 * wp + 4 * g + jj] * kds[jj];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        // P^T rows j = 16wp + li, k = i: column j of P, rows 32s..
        const Split8 A{lds_tr8s(&TPL[2][32 * s * kLT + 16 * wp], kLT, tid), lds_tr8s(&TPL[3][32 * s * kLT + 16 * wp], kLT, tid)};
        if constexpr (kExactDy) {
          dd = mma2(dd, A, lds_tr8s(dYm[0] + 32 * s * kLR, kLR, tid));
        } else {
          dd = mma3(dd, A, Split8{lds_tr8s(dYm[0] + 32 * s * kLR, kLR, tid), lds_tr8s(dYm[1] + 32 * s * kLR, kLR, tid)});
        }
      }
      put4(dDt[0], dDt[1], swz(li, 16 * wp + 4 * g, kLT), dd);
    } else {
      if (c > 0) load_kq(nxt, c - 1);
      // X = (diag(exp G) dY)^T Q for state columns 32 wp + 16 nt + li: A rows r = li, k = i (transposing read of
      // diag(exp G) dY), B = q rows i.
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        const int c0 = 32 * wp + 16 * nt;
        f32x4 x = zero4();
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const Split8 Ay{lds_tr8s(GdYm[0] + 32 * s * kLR, kLR, tid), lds_tr8s(GdYm[1] + 32 * s * kLR, kLR, tid)};
          x = mma2(x, Ay, lds_tr8s(&Qb[32 * s * kLDK + c0], kLDK, tid));
        }
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) Xs[(4 * g + jj) * kLX + c0 + li] = x[jj];
      }
    }
    __syncthreads();

    if (!side) {
      // dR = Tb^T dDelta for positions i = 16wp.. (A = Tb^T rows i, k = j); dv = dR.
      dr = zero4();
#pragma unroll
      for (int s = 0; s < 2; ++s) {  // (both k steps for every wave, as above)
        const int at = swz(li, 32 * s + 8 * g, kLT);
        dr = mma3(dr,
                  Split8{lds_tr8s(&TPL[0][32 * s * kLT + 16 * wp], kLT, tid),
                         lds_tr8s(&TPL[1][32 * s * kLT + 16 * wp], kLT, tid)},  // Tb^T rows i, k = j
                  Split8{lds8(dDt[0] + at), lds8(dDt[1] + at)});
      }
      const int i0 = 16 * wp + 4 * g;
      put4(GdRt[0], GdRt[1], swz(li, i0, kLT), -gam[i0] * dr[0], -gam[i0 + 1] * dr[1], -gam[i0 + 2] * dr[2],
           -gam[i0 + 3] * dr[3]);
    } else if (c > 0) {
      load_rest(nxt, c - 1);
    }
    __syncthreads();

    // dS <- exp(G_63) dS + X - (diag(exp G) dR)^T K for this wave's columns: A rows r = li, k = i.
    {
      const float glast = gam[kC - 1];
      const int col = 16 * w + li;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) dS[jj] = glast * dS[jj] + Xs[(4 * g + jj) * kLX + col];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int at = swz(li, 32 * s + 8 * g, kLT);
        const bf16x8 bk = lds_tr8s(&Kb[32 * s * kLDK + 16 * w], kLDK, tid);  // k rows 32s.., this lane's column
        dS = mma2(dS, Split8{lds8(GdRt[0] + at), lds8(GdRt[1] + at)}, bk);
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
  if (side && nch > 0) load_kq(pa, nch - 1), load_rest(pa, nch - 1);
  for (int c = nch - 1; c >= 0; c -= 2) {
    step(c, pa, pb, dr);
    if (c > 0) step(c - 1, pb, pa, dr);
  }
  if (!side && nch > 0) store_dv(0, dr);
  if (a.ds0) {
#pragma unroll
    for (int jj = 0; jj < 4; ++jj)
      a.ds0[((int64_t(n) * a.Hv + hv) * a.Dv + row0 + 4 * g + jj) * Dk + 16 * w + li] = dS[jj];
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
