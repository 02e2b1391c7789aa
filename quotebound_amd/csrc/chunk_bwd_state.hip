// Chunked design, kernel 3: the backward state pass. One block (12 waves) per (sequence, value head, kRows state
// rows: 16, or 32 when the 16-row blocks would not all fit on the device at once), over the chunks in reverse. With
// dS the cotangent of the block's rows of the chunk's end state (ds_out for the last chunk), per chunk, every product
// formed transposed so that a lane holds one position and four consecutive state rows (or one state row and four
// consecutive columns), for each 16-row tile of the block's rows:
//   store dS (the gradient kernel needs it)
//   dDelta^T = (dS K^T) D + dY^T P,  D = diag(exp(G_63 - G))      waves 0-3, positions 16w..16w+15: the chain
//   dR^T = dDelta^T T diag(beta);   dv = dR                        waves 0-3
//   X^T = Q^T (diag(exp G) dY)                                     waves 4-7, beside the chain (no dS in it)
//   dS^T <- exp(G_63) dS^T + X^T - K^T (diag(exp G) dR)            waves 0-3, state columns 32w..32w+31
// This is the adjoint of the forward state pass; together with the gradient kernel it reproduces the reference's
// backward (src/delta_grad.cpp:14-18). dS0 is what remains after the first chunk. T and P come ready from the prep
// kernel, packed; the products that contract over their rows read them through the transposing LDS read (tri_tr8).
// MFMA with split float32 operands as in the forward. Three barriers per chunk. The inputs of the next chunk (in the
// reverse sweep) are loaded and staged in LDS beside the chain by two groups, one wave of each per SIMD: waves 4-7
// the k and q rows (and X^T), waves 8-11 dy, the packed T and P and the per-position vectors; waves 0-3 touch global
// memory only to store dS and dv. Each group's loads and LDS writes go in windows where it would otherwise wait for
// the chain, and neither group's loads hold back the other's LDS writes. The three groups run loops of their own,
// with the same barriers, so that each loop holds only its own group's memory operations and the compiler's waits
// stay exact.
#include <type_traits>

#include "chunk_common.h"
#include "chunk_kernels.h"

namespace qbgdn {
namespace {

constexpr int kThreads = 768;  // waves 0-3 the chain, 4-7 k, q and X^T, 8-11 dy, T, P
// Row pitches (elements) of the swz-placed LDS matrices: 16 x an odd number.
constexpr int kLS = 144;  // dS [kRows][128]
constexpr int kLK = 144;  // k, q rows [64][128]
constexpr int kLX = 128 + 4;       // float32 X^T rows [kRows][..] (state row, then column)
constexpr int kTriUnits = 3 * 256;  // 16-byte units of a staged packed matrix (hi, lo: 640 used, the rest padding)
// dY, diag(exp G) dY, dDelta and -diag(exp G) dR ([64][kRows] each, positions as rows) side by side in one [64][kLW]
// matrix, at columns 0, kRows, 2 kRows and 3 kRows: a view at a column offset that is a multiple of 16 is swz-placed
// with the same pitch, so each keeps the conflict-free reads of a matrix of its own, without its own padding.
template <int kRows>
constexpr int kLW = kRows == 16 ? 80 : 144;

template <typename OutT, int kRows>
__global__ __launch_bounds__(kThreads) void chunk_bwd_state_kernel(ChunkArgs a) {
  constexpr int Dk = 128, kRT = kRows / 16, kLP = kLW<kRows>;
  constexpr int oY = 0, oGY = kRows, odD = 2 * kRows, oGR = 3 * kRows;  // column offsets in Wm
  static_assert(4 * kRows <= kLP, "dY, diag(exp G) dY, dDelta and -diag(exp G) dR side by side");
  constexpr bool kExactDy = std::is_same<OutT, bf16_t>::value;  // bf16 cotangents enter MFMA exactly
  __shared__ __align__(16) __bf16 dSm[2][kRows * kLS];            // dS rows, hi and lo
  __shared__ __align__(16) __bf16 Kb[2][kC * kLK];                // k rows, by chunk parity
  __shared__ __align__(16) __bf16 Qb[kC * kLK];                   // q rows
  __shared__ __align__(16) __bf16 Wm[2][kC * kLP];                // dY, diag(exp G) dY, dDelta, -diag(exp G) dR
  __shared__ __align__(16) __bf16 Tbp[kTriUnits * 8], Pp[kTriUnits * 8];  // packed T, P (hi then lo)
  __shared__ __align__(16) float Xs[kRows * kLX];
  __shared__ float Gs[2][3 * kC];  // exp G, D, beta, by chunk parity

  const int total = a.nblk * a.Hv * a.N;
  const StateItem item = state_item(a.tab, blockIdx.x, a.nblk, a.Hv, a.Hk, total);
  const int blk = item.blk, hv = item.hv, n = item.n;
  const int hk = hv / (a.Hv / a.Hk), row0 = kRows * blk;
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, li = lane & 15;
  // The wave index, made visibly uniform so that its branches are scalar and buffer resources stay in scalar
  // registers.
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wp = w & 3, ip = 16 * wp + li;  // position tile; the lane's position in products over positions
  const int u = tid & 255;                   // waves 4-11: thread index within the wave's group
  const Seq sq = seq_of(a.tab, n);
  const int nch = (sq.len + kC - 1) / kC;
  const OutT* dy = static_cast<const OutT*>(a.dy);
  OutT* dv = static_cast<OutT*>(a.dv);
  const int sk = a.Hk * Dk, sv = a.Hv * a.Dv;
  const int64_t srow = (int64_t(n) * a.Hv + hv) * a.Dv + row0 + li;  // the lane's state row in the first row tile

  if (w >= 4) {
    // Waves 4-11. One chunk's inputs, loaded a chunk ahead: (a) k and q rows (waves 4-7), staged while the chain
    // computes dR; (b) dy, the packed T and P, and exp G, D, beta (waves 8-11), staged after the chain's last use of
    // the previous ones. k, q, dy go through buffer resources that end at the sequence's last row, so rows past it
    // read as zeros without a branch; units past the packed matrices read as zeros and land in padding.
    struct GroupA {
      uint4 k[4], q[4];  // units u + 256 q4: row e / 16, columns 8 (e % 16) ..
    };
    struct GroupB {
      uint4 dy[kRT];        // row u / 4, state rows 16 rt + 4 (u % 4) .. + 3: raw bits (4 bf16 in .x, .y, or 4 float32)
      uint4 tb[3], p[3];    // packed T and P units u + 256 t
      float gam, dec, bet;  // of position lane (every wave loads all 64)
    };
    auto load_a = [&](GroupA& f, int c) {
      const int64_t tok = sq.tok0 + int64_t(c) * kC;
      const uint32_t L = uint32_t(min(kC, sq.len - c * kC));
      const auto kr = buffer_rsrc(a.k + tok * sk + hk * Dk, L * sk * 2);
      const auto qr = buffer_rsrc(a.q + tok * sk + hk * Dk, L * sk * 2);
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int e = u + 256 * q4;
        f.k[q4] = buf_ld16(kr, uint32_t((e >> 4) * sk + (e & 15) * 8) * 2);
      }
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int e = u + 256 * q4;
        f.q[q4] = buf_ld16(qr, uint32_t((e >> 4) * sk + (e & 15) * 8) * 2);
      }
    };
    auto load_b = [&](GroupB& f, int c) {
      const int64_t tok = sq.tok0 + int64_t(c) * kC;
      const uint32_t L = uint32_t(min(kC, sq.len - c * kC));
      const Tile* tl = a.tiles + ((sq.slot0 + c) * a.Hv + hv);
      const auto yr = buffer_rsrc(dy + tok * sv + hv * a.Dv + row0, L * sv * uint32_t(sizeof(OutT)));
#pragma unroll
      for (int rt = 0; rt < kRT; ++rt) {
        const uint32_t yo = uint32_t((u >> 2) * sv + 16 * rt + 4 * (u & 3));
        if constexpr (kExactDy) {
          const uint2 t2 = buf_ld8(yr, yo * 2);
          f.dy[rt] = uint4{t2.x, t2.y, 0u, 0u};
        } else {
          f.dy[rt] = buf_ld16(yr, yo * 4);
        }
      }
      const auto tr = buffer_rsrc(tl->t[0], 2 * kTri * 2), pr = buffer_rsrc(tl->p[0], 2 * kTri * 2);
#pragma unroll
      for (int t = 0; t < 3; ++t) f.tb[t] = buf_ld16(tr, uint32_t(u + 256 * t) * 16);
#pragma unroll
      for (int t = 0; t < 3; ++t) f.p[t] = buf_ld16(pr, uint32_t(u + 256 * t) * 16);
      const auto gr = buffer_rsrc(tl->gam, 3 * kC * 4);  // gam, dec, beta
      f.gam = buf_ld4(gr, uint32_t(lane) * 4), f.dec = buf_ld4(gr, uint32_t(kC + lane) * 4);
      f.bet = buf_ld4(gr, uint32_t(2 * kC + lane) * 4);
    };
    auto stage_a = [&](const GroupA& f, int b) {
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int e = u + 256 * q4, at = swz(e >> 4, (e & 15) * 8, kLK);
        *reinterpret_cast<uint4*>(Kb[b] + at) = f.k[q4];
        *reinterpret_cast<uint4*>(Qb + at) = f.q[q4];
      }
    };
    auto stage_b = [&](const GroupB& f, int b) {
      // dy's four values of row u / 4, as floats, and the same times exp G of that row (lane u / 4 of this wave
      // holds it).
      const int yt = u >> 2, yr4 = 4 * (u & 3);
      const float gy = __shfl(f.gam, yt);
#pragma unroll
      for (int rt = 0; rt < kRT; ++rt) {
        float yv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint4& d = f.dy[rt];
          const uint32_t x = kExactDy ? (j & 1 ? (&d.x)[j >> 1] & 0xffff0000u : (&d.x)[j >> 1] << 16) : (&d.x)[j];
          yv[j] = __uint_as_float(x);
        }
        put4(Wm[0], Wm[1], swz(yt, oY + 16 * rt + yr4, kLP), yv[0], yv[1], yv[2], yv[3]);
        put4(Wm[0], Wm[1], swz(yt, oGY + 16 * rt + yr4, kLP), gy * yv[0], gy * yv[1], gy * yv[2], gy * yv[3]);
      }
#pragma unroll
      for (int t = 0; t < 3; ++t) {
        *reinterpret_cast<uint4*>(Tbp + 8 * (u + 256 * t)) = f.tb[t];
        *reinterpret_cast<uint4*>(Pp + 8 * (u + 256 * t)) = f.p[t];
      }
      if (u < kC) Gs[b][u] = f.gam, Gs[b][kC + u] = f.dec, Gs[b][2 * kC + u] = f.bet;
    };
    // Per chunk c, with two register sets in turn: X^T for chunk c (its q and diag(exp G) dY were staged during
    // chunk c + 1); the inputs of chunk c - 1, loaded during chunk c + 1, to LDS; the loads of chunk c - 2 (clamped
    // at 0: the last chunks load chunk 0 again rather than branch).
    if (w < 8) {
      auto step = [&](int c, GroupA& cur, GroupA& nxt) {
        const int cs = max(c - 1, 0), cn = max(c - 2, 0);
        __syncthreads();
        load_a(nxt, cn);
        // X^T = Q^T (diag(exp G) dY) for state columns 32 wp + 16 t + 4g + jj, state row 16 rt + li: A = Q^T through
        // the transposing read of the q rows, B = diag(exp G) dY through the transposing read.
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          bf16x8 aq[2];
#pragma unroll
          for (int s = 0; s < 2; ++s) aq[s] = lds_tr8s(Qb + swz(32 * s, 32 * wp + 16 * t, kLK), kLK, lane);
#pragma unroll
          for (int rt = 0; rt < kRT; ++rt) {
            f32x4 x2[2];
#pragma unroll
            for (int s = 0; s < 2; ++s) {
              const int o = 32 * s * kLP + oGY + 16 * rt;
              x2[s] = mma2(zero4(), aq[s], Split8{lds_tr8s(Wm[0] + o, kLP, lane), lds_tr8s(Wm[1] + o, kLP, lane)});
            }
            *reinterpret_cast<f32x4*>(Xs + (16 * rt + li) * kLX + 32 * wp + 16 * t + 4 * g) = x2[0] + x2[1];
          }
        }
        __syncthreads();
        stage_a(cur, cs & 1);  // q's last readers (the X^T above) and k's (chunk c + 1) are a barrier back
        __syncthreads();
      };
      GroupA ga, gb;
      if (nch > 0) {
        load_a(ga, nch - 1);
        stage_a(ga, (nch - 1) & 1);
        load_a(ga, max(nch - 2, 0));
      }
      int c = nch - 1;
      for (; c >= 1; c -= 2) {
        step(c, ga, gb);
        step(c - 1, gb, ga);
      }
      if (c == 0) step(0, ga, gb);
    } else {
      auto step = [&](int c, GroupB& cur, GroupB& nxt) {
        const int cs = max(c - 1, 0), cn = max(c - 2, 0);
        __syncthreads();
        __syncthreads();
        load_b(nxt, cn);
        __syncthreads();
        // The chain's last readers of dY, T and P, and X^T's of diag(exp G) dY, were before this barrier.
        stage_b(cur, cs & 1);
      };
      GroupB ga, gb;
      if (nch > 0) {
        load_b(ga, nch - 1);
        stage_b(ga, (nch - 1) & 1);
        load_b(ga, max(nch - 2, 0));
      }
      int c = nch - 1;
      for (; c >= 1; c -= 2) {
        step(c, ga, gb);
        step(c - 1, gb, ga);
      }
      if (c == 0) step(0, ga, gb);
    }
    return;
  }

  // Waves 0-3: the recurrence. dS tile (rt, t) holds dS[16 rt + li][32 wp + 16 t + 4 g + jj]. (ds_out and ds0 need
  // only 4-byte alignment: one element at a time.)
  f32x4 dS[kRT][2];
#pragma unroll
  for (int rt = 0; rt < kRT; ++rt) dS[rt][0] = zero4(), dS[rt][1] = zero4();
  if (a.ds_out) {
#pragma unroll
    for (int rt = 0; rt < kRT; ++rt)
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj)
          dS[rt][t][jj] = a.ds_out[(srow + 16 * rt) * Dk + 32 * wp + 16 * t + 4 * g + jj];
  }
  for (int c = nch - 1; c >= 0; --c) {
    const int64_t slot = sq.slot0 + c, tok = sq.tok0 + int64_t(c) * kC;
    const uint32_t L = uint32_t(min(kC, sq.len - c * kC));
    const int b = c & 1;
    {  // dS to the workspace and, split, to LDS (its last readers are two barriers back)
      const auto out = buffer_rsrc(a.dsend + ((slot * a.Hv + hv) * a.Dv + row0) * Dk, kRows * Dk * 4);
#pragma unroll
      for (int rt = 0; rt < kRT; ++rt)
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int col = 32 * wp + 16 * t + 4 * g;
          put4(dSm[0], dSm[1], swz(16 * rt + li, col, kLS), dS[rt][t]);
          BufIO<float>::st4(out, uint32_t((16 * rt + li) * Dk + col), dS[rt][t]);
        }
    }
    __syncthreads();

    {  // dDelta^T at state rows 16 rt + 4g + jj, position ip = (dS K^T) D + dY^T P
      f32x4 xh[kRT], xl[kRT], z[kRT];  // independent chains
#pragma unroll
      for (int rt = 0; rt < kRT; ++rt) xh[rt] = zero4(), xl[rt] = zero4(), z[rt] = zero4();
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const bf16x8 bk = lds8(Kb[b] + swz(ip, 32 * s + 8 * g, kLK));
#pragma unroll
        for (int rt = 0; rt < kRT; ++rt) {
          const int at = swz(16 * rt + li, 32 * s + 8 * g, kLS);
          xh[rt] = mma(xh[rt], lds8(dSm[0] + at), bk);
          xl[rt] = mma(xl[rt], lds8(dSm[1] + at), bk);
        }
      }
#pragma unroll
      for (int s = 0; s < 2; ++s) {  // dY^T P: A = dY^T through the transposing read, B = P's column ip
        const Split8 B{tri_tr8(Pp, 32 * s, wp, lane), tri_tr8(Pp + kTri, 32 * s, wp, lane)};
#pragma unroll
        for (int rt = 0; rt < kRT; ++rt) {
          const int o = 32 * s * kLP + oY + 16 * rt;
          if constexpr (kExactDy) {
            z[rt] = mma2(z[rt], lds_tr8s(Wm[0] + o, kLP, lane), B);
          } else {
            z[rt] = mma3(z[rt], Split8{lds_tr8s(Wm[0] + o, kLP, lane), lds_tr8s(Wm[1] + o, kLP, lane)}, B);
          }
        }
      }
      const float dec = Gs[b][kC + ip];
#pragma unroll
      for (int rt = 0; rt < kRT; ++rt) {
        const f32x4 dd = dec * (xh[rt] + xl[rt]) + z[rt];
        put4(Wm[0], Wm[1], swz(ip, odD + 16 * rt + 4 * g, kLP), dd);
      }
    }
    __syncthreads();

    {  // dR^T = dDelta^T T diag(beta): A = dDelta^T through the transposing read, B = T's column ip; dv = dR
      Split8 TB[2];
#pragma unroll
      for (int s = 0; s < 2; ++s) TB[s] = Split8{tri_tr8(Tbp, 32 * s, wp, lane), tri_tr8(Tbp + kTri, 32 * s, wp, lane)};
      const float bet = Gs[b][2 * kC + ip], ngam = -Gs[b][ip];
      // Positions past the chunk's end fall past the resource and are dropped.
      const auto vr = buffer_rsrc(dv + tok * sv + hv * a.Dv + row0, L * sv * uint32_t(sizeof(OutT)));
#pragma unroll
      for (int rt = 0; rt < kRT; ++rt) {
        f32x4 d2[2];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const int o = 32 * s * kLP + odD + 16 * rt;
          d2[s] = mma3(zero4(), Split8{lds_tr8s(Wm[0] + o, kLP, lane), lds_tr8s(Wm[1] + o, kLP, lane)}, TB[s]);
        }
        const f32x4 dr = bet * (d2[0] + d2[1]);
        BufIO<OutT>::st4(vr, uint32_t(ip * sv + 16 * rt + 4 * g), dr);
        put4(Wm[0], Wm[1], swz(ip, oGR + 16 * rt + 4 * g, kLP), ngam * dr);
      }
    }
    __syncthreads();

    // dS^T <- exp(G_63) dS^T + X^T + K^T (-diag(exp G) dR): A = K^T rows 32 wp + 16 t + li through the transposing
    // read, B = -diag(exp G) dR through the transposing read.
    const float glast = Gs[b][kC - 1];
#pragma unroll
    for (int rt = 0; rt < kRT; ++rt)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const f32x4 x = *reinterpret_cast<const f32x4*>(Xs + (16 * rt + li) * kLX + 32 * wp + 16 * t + 4 * g);
        dS[rt][t] = glast * dS[rt][t] + x;
      }
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      bf16x8 KA[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) KA[t] = lds_tr8s(Kb[b] + swz(32 * s, 32 * wp + 16 * t, kLK), kLK, lane);
#pragma unroll
      for (int rt = 0; rt < kRT; ++rt) {
        const int o = 32 * s * kLP + oGR + 16 * rt;
        const Split8 B{lds_tr8s(Wm[0] + o, kLP, lane), lds_tr8s(Wm[1] + o, kLP, lane)};
#pragma unroll
        for (int t = 0; t < 2; ++t) dS[rt][t] = mma2(dS[rt][t], KA[t], B);
      }
    }
  }
  if (a.ds0) {
#pragma unroll
    for (int rt = 0; rt < kRT; ++rt)
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) a.ds0[(srow + 16 * rt) * Dk + 32 * wp + 16 * t + 4 * g + jj] = dS[rt][t][jj];
  }
}

}  // namespace

hipError_t launch_chunk_bwd_state(const ChunkArgs& a, bool out_bf16, hipStream_t s) {
  const int total = a.nblk * a.Hv * a.N;
  const bool r32 = a.Dv == 32 * a.nblk;  // 32 state rows per block (else 16)
  void (*k)(ChunkArgs) = out_bf16 ? (r32 ? chunk_bwd_state_kernel<bf16_t, 32> : chunk_bwd_state_kernel<bf16_t, 16>)
                                  : (r32 ? chunk_bwd_state_kernel<float, 32> : chunk_bwd_state_kernel<float, 16>);
  hipLaunchKernelGGL(k, dim3(total), dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace qbgdn
