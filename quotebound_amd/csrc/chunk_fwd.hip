// Chunked design, kernel 2: the forward state pass. One block (8 waves) per (sequence, value head, 16 state rows),
// sequential over the sequence's chunks; rows of the state evolve independently (reference src/delta_grad.cpp:13),
// so a 16-row block needs no other block. Per chunk, with S the block's rows of the state at the chunk start:
//   write S to the chunk's checkpoint slot (the reference's ckpt, src/delta_grad.cpp:172-181)
//   KS = K S^T, R = V - diag(exp G) KS, Delta = Tb R             waves 0-3, positions 16w..16w+15: the chain
//   QS = Q S^T, Y = diag(exp G) QS + P Delta                      waves 4-7, positions 16(w-4)..: off the chain
//   S <- exp(G_63) S + (diag(exp(G_63 - G)) Delta)^T K            every wave: state columns 16w..16w+15
// Two waves share each SIMD, one on the chain and one beside it. Tb and P come ready from the prep kernel (each
// wave loads its rows as MFMA A operands). All products run on v_mfma_f32_16x16x32_bf16; float32 operands (S, R,
// Delta, Tb, P) are split into bf16 hi + lo pairs so the state keeps float32 accuracy, while k, q, v enter exactly.
// The next chunk's inputs are loaded into registers while the current chunk computes.
#include "chunk_common.h"
#include "chunk_kernels.h"

namespace qbgdn {
namespace {

constexpr int kThreads = 512;
// Row pitches (elements) of the swz-placed LDS matrices: 16 x an odd number.
constexpr int kLDK = 144;  // k, q rows [64][128]
constexpr int kLDC = 80;   // [16][64]: R^T, Delta^T, (D Delta)^T
constexpr int kLR = 48;    // [128][16]: S^T (state rows as columns)

template <typename OutT>
__global__ __launch_bounds__(kThreads) void chunk_fwd_kernel(ChunkArgs a) {
  constexpr int Dk = 128;
  // Every matrix is placed by swz and stored once, hi and lo: row reads and transposing reads both come free of
  // bank conflicts.
  __shared__ __align__(16) __bf16 Kb[kC * kLDK], Qb[kC * kLDK];
  __shared__ __align__(16) __bf16 St[2][128 * kLR];                       // S^T [c][r]
  __shared__ __align__(16) __bf16 Rt[2][16 * kLDC], Dt[2][16 * kLDC];  // [r][i]
  __shared__ __align__(16) __bf16 DDt[2][16 * kLDC];
  __shared__ float Vs[kC][16];
  __shared__ float gam[kC], dec[kC];

  const int total = a.nblk * a.Hv * a.N;
  const int wid = xcd_remap(blockIdx.x, total);
  const int blk = wid % a.nblk, hv = (wid / a.nblk) % a.Hv, n = wid / (a.nblk * a.Hv);
  const int hk = hv / (a.Hv / a.Hk), row0 = 16 * blk;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, li = lane & 15;
  const int wp = w & 3;            // position tile
  const bool side = w >= 4;        // off the chain: Q S^T and Y
  const int i0 = 16 * wp + 4 * g;  // first of the lane's accumulator positions
  const Seq sq = seq_of(a.tab, n);
  const int nch = (sq.len + kC - 1) / kC;
  OutT* y = static_cast<OutT*>(a.y);
  const int sk = a.Hk * Dk, sv = a.Hv * a.Dv;  // token strides of k/q and v/y

  // State: wave w holds rows 4g + jj, columns 16w + li.
  f32x4 S;
#pragma unroll
  for (int jj = 0; jj < 4; ++jj)
    S[jj] = a.s0 ? a.s0[((int64_t(n) * a.Hv + hv) * a.Dv + row0 + 4 * g + jj) * Dk + 16 * w + li] : 0.f;

  // One chunk's inputs, loaded into registers a chunk ahead: k and q rows by waves 0-3, right after they have
  // written the state (they then wait for waves 4-7 anyway); v, exp G, D by waves 4-7 after the barrier; each wave's
  // own A operand rows. k, q, v go through buffer resources that end at the sequence's last row, so rows past it
  // read as zeros without a branch.
  struct Pre {
    uint4 k[4], q[4];  // waves 0-3, thread e = tid + 256 q4: row e / 16, columns 8 (e % 16) ..
    uint16_t v[4];     // waves 4-7, e = tid - 256 + 256 q4: v row e / 16, state row e % 16
    bf16x8 f[4];       // waves 0-3: Tb rows 16 wp + li; waves 4-7: P rows (k = 8g.., two k steps, hi and lo)
    float gd;          // waves 4-5: exp G (tid - 256 < 64), then D = exp(G_63 - G)
  };
  auto prefetch = [&](Pre& f, int c) {
    const int64_t slot = sq.slot0 + c, tok = sq.tok0 + int64_t(c) * kC;
    const uint32_t L = uint32_t(min(kC, sq.len - c * kC));
    const auto kr = buffer_rsrc(a.k + tok * sk + hk * Dk, L * sk * 2);
    const auto qr = buffer_rsrc(a.q + tok * sk + hk * Dk, L * sk * 2);
    const auto vr = buffer_rsrc(a.v + tok * sv + hv * a.Dv + row0, L * sv * 2);
    const Tile* tl = a.tiles + (slot * a.Hv + hv);
    if (!side) {
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int e = tid + 256 * q4, t = e >> 4, c8 = (e & 15) * 8;
        f.k[q4] = buf_ld16(kr, uint32_t(t * sk + c8) * 2);
        f.q[q4] = buf_ld16(qr, uint32_t(t * sk + c8) * 2);
      }
    } else {
      const int u = tid - 256;
      f.gd = (u < kC ? tl->gam : tl->dec)[u & (kC - 1)];
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int e = u + 256 * q4, t = e >> 4;
        f.v[q4] = buf_ld2(vr, uint32_t(t * sv + (e & 15)) * 2);
      }
    }
    const auto mr = buffer_rsrc(side ? tl->p[0] : tl->tb[0], 2 * kTri * 2);  // hi, then lo
    const int ar = 16 * wp + li;
    f.f[0] = tri_ld8(mr, 0, ar, 8 * g), f.f[1] = tri_ld8(mr, kTri, ar, 8 * g);
    f.f[2] = tri_ld8(mr, 0, ar, 32 + 8 * g), f.f[3] = tri_ld8(mr, kTri, ar, 32 + 8 * g);  // zeros for rows < 32
  };

  // y of a chunk (waves 4-7) is stored during the next chunk, after that chunk's inputs are staged, so no wait for
  // the staged loads ever covers these stores.
  auto store_y = [&](int c, const f32x4& yacc) {
    const int64_t tok = sq.tok0 + int64_t(c) * kC;
    const uint32_t L = uint32_t(min(kC, sq.len - c * kC));
    // Rows i >= L fall past the resource and are dropped.
    const auto yr = buffer_rsrc(y + tok * sv + hv * a.Dv + row0, L * sv * uint32_t(sizeof(OutT)));
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) BufIO<OutT>::st(yr, uint32_t((i0 + jj) * sv + li), yacc[jj]);
  };

  auto step = [&](int c, Pre& f, Pre& nxt, f32x4& yacc) {
    const int64_t slot = sq.slot0 + c;
    __syncthreads();  // the previous chunk's readers of LDS are done
    // Stage the chunk first: the waits for its loads then come before this chunk's own stores.
    if (!side) {
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int e = tid + 256 * q4, t = e >> 4, c8 = (e & 15) * 8;
        *reinterpret_cast<uint4*>(&Kb[swz(t, c8, kLDK)]) = f.k[q4];
        *reinterpret_cast<uint4*>(&Qb[swz(t, c8, kLDK)]) = f.q[q4];
      }
    } else {
      const int u = tid - 256;
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int e = u + 256 * q4;
        Vs[e >> 4][e & 15] = bf16_to_f32(f.v[q4]);
      }
      if (u < kC)
        gam[u] = f.gd;
      else if (u < 2 * kC)
        dec[u - kC] = f.gd;
    }
    // The A operands are consumed later in the step: take them here, so their waits are here too.
#pragma unroll
    for (int u = 0; u < 4; ++u) asm volatile("" : "+v"(f.f[u]));
    if (side && c > 0) store_y(c - 1, yacc);
    {  // S to the checkpoint and, split, to LDS.
      const auto ck = a.ckpt ? buffer_rsrc(a.ckpt + ((slot * a.Hv + hv) * a.Dv + row0) * Dk, 16 * Dk * 4)
                             : buffer_rsrc(a.s0, 0);
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int r = 4 * g + jj, col = 16 * w + li;
        const float x = S[jj];
        BufIO<float>::st(ck, uint32_t(r * Dk + col), x);
      }
      put4(St[0], St[1], swz(16 * w + li, 4 * g, kLR), S);  // S^T: this lane's column, its four rows
    }
    if (!side && c + 1 < nch) prefetch(nxt, c + 1);
    __syncthreads();
    if (side && c + 1 < nch) prefetch(nxt, c + 1);

    // K S^T (waves 0-3) or Q S^T (waves 4-7) for positions i0 + jj, state row li.
    f32x4 xs = zero4();
    {
      const __bf16* M = side ? Qb : Kb;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const bf16x8 am = lds8(M + swz(16 * wp + li, 32 * s + 8 * g, kLDK));
        // B = S rows r (n), k = c: the transposing read of S^T
        xs = mma(mma(xs, am, lds_tr8s(St[0] + 32 * s * kLR, kLR, tid)), am, lds_tr8s(St[1] + 32 * s * kLR, kLR, tid));
      }
    }
    if (!side) {
      f32x4 r;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) r[jj] = Vs[i0 + jj][li] - gam[i0 + jj] * xs[jj];
      put4(Rt[0], Rt[1], swz(li, i0, kLDC), r);
    }
    __syncthreads();

    if (!side) {  // Delta = Tb R for positions i0 + jj
      f32x4 dl = zero4();
      // Both k steps for every wave: Tb's entries above the diagonal are zeros, and the waves that need both set
      // the pace, so skipping would only add branches.
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int at = swz(li, 32 * s + 8 * g, kLDC);
        dl = mma3(dl, Split8{f.f[2 * s], f.f[2 * s + 1]}, Split8{lds8(Rt[0] + at), lds8(Rt[1] + at)});
      }
      f32x4 dd;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) dd[jj] = dec[i0 + jj] * dl[jj];
      put4(Dt[0], Dt[1], swz(li, i0, kLDC), dl);
      put4(DDt[0], DDt[1], swz(li, i0, kLDC), dd);
    }
    __syncthreads();

    // S <- exp(G_63) S + (D Delta)^T K: this wave's columns 16w + li, rows 4g + jj.
    {
      const float glast = gam[kC - 1];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) S[jj] *= glast;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int at = swz(li, 32 * s + 8 * g, kLDC);
        const Split8 A{lds8(DDt[0] + at), lds8(DDt[1] + at)};
        S = mma2(S, A, lds_tr8s(Kb + 32 * s * kLDK + 16 * w, kLDK, tid));  // K rows 32s.., this lane's state column
      }
    }
    if (side) {  // Y = diag(exp G) QS + P Delta for positions i0 + jj (P is zero above the diagonal)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) yacc[jj] = gam[i0 + jj] * xs[jj];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int at = swz(li, 32 * s + 8 * g, kLDC);
        yacc = mma3(yacc, Split8{f.f[2 * s], f.f[2 * s + 1]}, Split8{lds8(Dt[0] + at), lds8(Dt[1] + at)});
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
  if (side && nch > 0) store_y(nch - 1, yacc);
  if (a.s_out) {
#pragma unroll
    for (int jj = 0; jj < 4; ++jj)
      a.s_out[((int64_t(n) * a.Hv + hv) * a.Dv + row0 + 4 * g + jj) * Dk + 16 * w + li] = S[jj];
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
