// Chunked design, kernel 2: the forward state pass. One block (4 waves) per (sequence, value head, 16 state rows),
// sequential over the sequence's chunks; rows of the state evolve independently (reference src/delta_grad.cpp:13),
// so a 16-row block needs no other block. Per chunk, with S the block's rows of the state at the chunk start:
//   write S to the chunk's checkpoint slot (the reference's ckpt, src/delta_grad.cpp:172-181)
//   KS = K S^T, QS = Q S^T                        [64 x 16]   wave w: positions 16w..16w+15
//   R = V - diag(exp G) KS;  Delta = Tb R
//   S <- exp(G_63) S + (diag(exp(G_63 - G)) Delta)^T K        wave w: state columns 32w..32w+31
//   Y = diag(exp G) QS + P Delta
// Tb and P come ready from the prep kernel (each wave loads its rows as MFMA A operands). All products run on v_mfma_f32_16x16x32_bf16; float32 operands (S, R,
// Delta, Tb, P) are split into bf16 hi + lo pairs so the state keeps float32 accuracy, while k, q, v enter exactly.
// The next chunk's inputs are loaded into registers while the current chunk computes.
#include "chunk_common.h"
#include "chunk_kernels.h"

namespace qbgdn {
namespace {

constexpr int kThreads = 256;
constexpr int kLDK = 144;  // bf16 row stride for Dk = 128 (rows 0..3 of a transposing read on distinct banks)
constexpr int kLDC = kC + kPadB;   // bf16 row stride for 64 positions

template <typename OutT>
__global__ __launch_bounds__(kThreads) void chunk_fwd_kernel(ChunkArgs a) {
  constexpr int Dk = 128;
  __shared__ __bf16 Kb[kC][kLDK], Qb[kC][kLDK];
  __shared__ __bf16 Sh[16][kLDK], Sl[16][kLDK];
  __shared__ __bf16 Rth[16][kLDC], Rtl[16][kLDC], Dth[16][kLDC], Dtl[16][kLDC], DDth[16][kLDC], DDtl[16][kLDC];
  __shared__ float Vs[kC][16];
  __shared__ float gam[kC], dec[kC];

  const int total = a.nblk * a.Hv * a.N;
  const int wid = xcd_remap(blockIdx.x, total);
  const int blk = wid % a.nblk, hv = (wid / a.nblk) % a.Hv, n = wid / (a.nblk * a.Hv);
  const int hk = hv / (a.Hv / a.Hk), row0 = 16 * blk;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, li = lane & 15;
  const Seq sq = seq_of(a.tab, n);
  const int nch = (sq.len + kC - 1) / kC;
  OutT* y = static_cast<OutT*>(a.y);
  const int sk = a.Hk * Dk, sv = a.Hv * a.Dv;  // token strides of k/q and v/y

  // State block: wave w holds rows 4g + jj, columns 32w + 16nt + li.
  f32x4 S[2];
#pragma unroll
  for (int nt = 0; nt < 2; ++nt)
#pragma unroll
    for (int jj = 0; jj < 4; ++jj)
      S[nt][jj] = a.s0 ? a.s0[((int64_t(n) * a.Hv + hv) * a.Dv + row0 + 4 * g + jj) * Dk + 32 * w + 16 * nt + li]
                       : 0.f;

  // One chunk's inputs, loaded into registers a chunk ahead: k and q rows (thread e of [0, 1024) in steps of 256
  // covers row e / 16, columns 8 (e % 16)), v (row e / 16, state row e % 16), exp G, D, and the wave's A operands,
  // Tb rows 16w + li and P rows 16w + li (k = 8g.., two k steps, hi and lo). k, q, v are read through buffer
  // resources that end at the sequence's last row, so rows past it read as zeros without a branch.
  struct Pre {
    uint4 k[4], q[4];
    bf16x8 t[4], p[4];
    uint16_t v[4];
    float gam, dec;
  };
  auto prefetch = [&](Pre& f, int c) {
    const int64_t slot = sq.slot0 + c, tok = sq.tok0 + int64_t(c) * kC;
    const uint32_t L = uint32_t(min(kC, sq.len - c * kC));
    const auto kr = buffer_rsrc(a.k + tok * sk + hk * Dk, L * sk * 2);
    const auto qr = buffer_rsrc(a.q + tok * sk + hk * Dk, L * sk * 2);
    const auto vr = buffer_rsrc(a.v + tok * sv + hv * a.Dv + row0, L * sv * 2);
    const Tile* tl = a.tiles + (slot * a.Hv + hv);
    f.gam = tl->gam[tid & (kC - 1)], f.dec = tl->dec[tid & (kC - 1)];
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int e = tid + kThreads * q4, t = e >> 4, c8 = (e & 15) * 8;
      f.k[q4] = buf_ld16(kr, uint32_t(t * sk + c8) * 2);
      f.q[q4] = buf_ld16(qr, uint32_t(t * sk + c8) * 2);
      f.v[q4] = buf_ld2(vr, uint32_t(t * sv + (e & 15)) * 2);
    }
    const int ar = (16 * w + li) * kC + 8 * g;
    f.t[0] = gld8(tl->tb_hi + ar), f.t[1] = gld8(tl->tb_lo + ar), f.t[2] = gld8(tl->tb_hi + ar + 32),
    f.t[3] = gld8(tl->tb_lo + ar + 32);
    f.p[0] = gld8(tl->p_hi + ar), f.p[1] = gld8(tl->p_lo + ar), f.p[2] = gld8(tl->p_hi + ar + 32),
    f.p[3] = gld8(tl->p_lo + ar + 32);
  };

  // y of a chunk is stored during the next chunk (after that chunk's inputs are staged), so no wait for the
  // staged loads ever covers these stores.
  auto store_y = [&](int c, const f32x4& yacc) {
    const int64_t tok = sq.tok0 + int64_t(c) * kC;
    const uint32_t L = uint32_t(min(kC, sq.len - c * kC));
    // Rows i >= L fall past the resource and are dropped.
    const auto yr = buffer_rsrc(y + tok * sv + hv * a.Dv + row0, L * sv * uint32_t(sizeof(OutT)));
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) BufIO<OutT>::st(yr, uint32_t((16 * w + 4 * g + jj) * sv + li), yacc[jj]);
  };

  auto step = [&](int c, Pre& f, Pre& nxt, f32x4& yacc) {
    const int64_t slot = sq.slot0 + c;
    __syncthreads();  // the previous chunk's readers of LDS are done
    // Stage the chunk first: the waits for its loads then come before this chunk's own stores.
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int e = tid + kThreads * q4, t = e >> 4, c8 = (e & 15) * 8;
      *reinterpret_cast<uint4*>(&Kb[t][c8]) = f.k[q4];
      *reinterpret_cast<uint4*>(&Qb[t][c8]) = f.q[q4];
      Vs[t][e & 15] = bf16_to_f32(f.v[q4]);
    }
    if (tid < kC) gam[tid] = f.gam, dec[tid] = f.dec;
    // The A operands are consumed later in the step: take them here, so their waits are here too.
#pragma unroll
    for (int u = 0; u < 4; ++u) asm volatile("" : "+v"(f.t[u]), "+v"(f.p[u]));
    if (c > 0) store_y(c - 1, yacc);
    {
      const auto ck = a.ckpt ? buffer_rsrc(a.ckpt + ((slot * a.Hv + hv) * a.Dv + row0) * Dk, 16 * Dk * 4)
                             : buffer_rsrc(a.s0, 0);
#pragma unroll
      for (int nt = 0; nt < 2; ++nt)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int r = 4 * g + jj, col = 32 * w + 16 * nt + li;
          const float x = S[nt][jj];
          BufIO<float>::st(ck, uint32_t(r * Dk + col), x);
          const __bf16 h = (__bf16)x;
          Sh[r][col] = h;
          Sl[r][col] = (__bf16)(x - (float)h);
        }
    }
    __syncthreads();
    if (c + 1 < nch) prefetch(nxt, c + 1);

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

    // Delta = Tb R for positions 16w..
    f32x4 dl = zero4();
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const Split8 B{lds8(&Rth[li][32 * s + 8 * g]), lds8(&Rtl[li][32 * s + 8 * g])};
      dl = mma3(dl, Split8{f.t[2 * s], f.t[2 * s + 1]}, B);
    }
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int i = 16 * w + 4 * g + jj;
      const float x = dl[jj], xd = dec[i] * dl[jj];
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
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const Split8 A{lds8(&DDth[li][32 * s + 8 * g]), lds8(&DDtl[li][32 * s + 8 * g])};
        S[nt] = mma2(S[nt], A, lds_tr8(&Kb[32 * s][32 * w + 16 * nt], kLDK, tid));  // K rows 32s.., this lane's state column
      }
    }

    // Y = diag(exp G) QS + P Delta for positions i = 16w.. (P is zero above the diagonal).
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) yacc[jj] = gam[16 * w + 4 * g + jj] * qs[jj];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      if (32 * s <= 16 * w + 15) {
        const Split8 B{lds8(&Dth[li][32 * s + 8 * g]), lds8(&Dtl[li][32 * s + 8 * g])};
        yacc = mma3(yacc, Split8{f.p[2 * s], f.p[2 * s + 1]}, B);
      }
    }
  };

  // Two register sets in turn: chunk c computes from one while chunk c + 1 loads into the other.
  Pre pa, pb;
  f32x4 yacc = zero4();
  if (nch > 0) prefetch(pa, 0);
  for (int c = 0; c < nch; c += 2) {
    step(c, pa, pb, yacc);
    if (c + 1 < nch) step(c + 1, pb, pa, yacc);
  }
  if (nch > 0) store_y(nch - 1, yacc);
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
