// Chunked design, kernel 2: the forward state pass. One block (12 waves) per (sequence, value head, kRows state
// rows: 16, or 32 when the 16-row blocks would not all fit on the device at once), sequential over the sequence's
// chunks; rows of the state evolve independently (reference src/delta_grad.cpp:13), so a block needs no other block.
// Per chunk, with S the block's rows of the state at the chunk start, every product is formed transposed, so that a
// lane holds one position i and four consecutive state rows r (or one state row and four consecutive columns), for
// each 16-row tile of the block's rows:
//   write S to LDS and to the chunk's checkpoint slot (the reference's ckpt, src/delta_grad.cpp:172-181)
//   R^T = (V^T - (S K^T) diag(exp G)) diag(beta), and S Q^T        waves 4-7, positions 16(w-4)..
//   Delta^T = R^T T^T                                              waves 0-3, positions 16w..16w+15
//   S^T <- exp(G_63) S^T + K^T (D Delta),  D = diag(exp(G_63 - G)) waves 0-3, state columns 32w..32w+31
//   Y^T = (S Q^T) diag(exp G) + Delta^T P^T                        waves 4-7: off the chain
// Three barriers per chunk. Waves 0-3 carry the state and touch no global memory but the checkpoint stores.
// Waves 4-7 read S from LDS once for both S K^T and S Q^T, and form y from LDS. Waves 8-11 load every input two
// chunks ahead, each wave load reading whole cache lines, and stage them in LDS: the chain's k rows, packed T, v,
// exp G, D and beta (two buffers, by chunk parity), the output group's q rows and packed P (one buffer each); K^T for
// the state update comes from the staged k rows through the transposing read. The loads and the LDS writes are
// spread over the chain's phases and the work over two groups, so that neither group, nor the CU's vector memory
// path or LDS, holds the chain at its barriers. Each group runs a loop of its own, so that each loop holds only its
// own group's memory operations: the compiler's waits stay exact and none covers a load issued for a later chunk.
// All products run on v_mfma_f32_16x16x32_bf16; float32 operands (S, R, Delta, T, P) are split into bf16 hi + lo
// pairs so the state keeps float32 accuracy, while k, q, v enter exactly.
#include "chunk_common.h"
#include "chunk_kernels.h"

namespace qbgdn {
namespace {

constexpr int kThreads = 768;  // waves 0-3 the chain, 4-7 the output, 8-11 the staging
// Row pitches (elements) of the swz-placed LDS matrices: 16 x an odd number.
constexpr int kLS = 144;  // S [kRows][128]
constexpr int kLK = 144;  // K [64][128]
constexpr int kTbUnits = 3 * 256;  // 16-byte units of a staged packed T (hi, lo: 640 used, the rest padding)
// R, Delta and D Delta ([64][kRows] each, positions as rows) side by side in one [64][kLW] matrix, at columns 0,
// kRows and 2 kRows: a view at a column offset that is a multiple of 16 is swz-placed with the same pitch, so each
// keeps the conflict-free reads of a matrix of its own, without its own padding.
template <int kRows>
constexpr int kLW = kRows == 16 ? 48 : 112;

__device__ __forceinline__ float bf16_lo(uint32_t x) { return __uint_as_float(x << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t x) { return __uint_as_float(x & 0xffff0000u); }

template <typename OutT, int kRows>
__global__ __launch_bounds__(kThreads) void chunk_fwd_kernel(ChunkArgs a) {
  constexpr int Dk = 128, kRT = kRows / 16, kLP = kLW<kRows>;
  constexpr int oR = 0, oD = kRows, oDD = 2 * kRows;  // column offsets in Wm
  static_assert(3 * kRows <= kLP, "R, Delta and D Delta side by side");
  // Every matrix is placed by swz and stored once, hi and lo: row reads and transposing reads both come free of
  // bank conflicts. The staged inputs have two buffers, by chunk parity.
  __shared__ __align__(16) __bf16 Sm[2][kRows * kLS];
  __shared__ __align__(16) __bf16 Wm[2][kC * kLP];  // R, Delta, D Delta
  __shared__ __align__(16) __bf16 Kb[2][kC * kLK];
  __shared__ __align__(16) __bf16 Tbp[2][kTbUnits * 8];  // packed T (tri_off), hi then lo
  __shared__ __align__(16) bf16_t Vs[2][256 * 8];        // v [64][kRows] (with 16 rows, units 128.. padding)
  __shared__ __align__(16) float Gs[2][256];             // exp G [64], D [64], beta [64] (the rest padding)
  // The output group's operands, one buffer each: q rows (written after the chunk's S Q^T, read in the next) and
  // packed P (written after the previous chunk's y, read in this chunk's).
  __shared__ __align__(16) __bf16 Qb[kC * kLK];
  __shared__ __align__(16) __bf16 Pb[kTbUnits * 8];

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
  OutT* y = static_cast<OutT*>(a.y);
  const int sk = a.Hk * Dk, sv = a.Hv * a.Dv;  // token strides of k/q and v/y
  const int64_t srow = (int64_t(n) * a.Hv + hv) * a.Dv + row0 + li;  // the lane's state row in the first row tile

  // Waves 8-11 (the staging group) load each chunk's inputs two chunks ahead, in rows of 16-byte units that a wave
  // reads whole (every cache line it touches in full), and stage them in LDS: k, packed T, v and the per-position
  // vectors for the chain and the output group's R (two buffers, by chunk parity), q and packed P for waves 4-7 (the
  // output group), which then read no global memory. k, q, v go through buffer resources that end at the sequence's
  // last row, so rows past it read as zeros without a branch; units past the packed matrices, v or the three
  // per-position vectors read as zeros, and the waves whose units are all past them skip those LDS writes.
  struct Stage {
    uint4 k[4];   // k units u + 256 q4: row e / 16, columns 8 (e % 16) ..
    uint4 q[4];   // q, the same units
    uint4 tb[3];  // packed T units u + 256 t
    uint4 p[3];   // packed P units u + 256 t
    uint4 v;      // v unit u: row u / (kRows / 8), state rows 8 (u % (kRows / 8)) ..
    float gd;     // exp G_u (u < 64), D_(u - 64) (u < 128), beta_(u - 128) (u < 192)
  };
  // The loads in two parts, issued in two of the chain's phases so that the CU's vector memory path is not asked
  // for a whole chunk's bytes at once: k and packed T, then q, packed P, v and the per-position vectors.
  auto load1 = [&](Stage& st, int c) {
    const int64_t slot = sq.slot0 + c, tok = sq.tok0 + int64_t(c) * kC;
    const uint32_t L = uint32_t(min(kC, sq.len - c * kC));
    const Tile* tl = a.tiles + (slot * a.Hv + hv);
    const auto kr = buffer_rsrc(a.k + tok * sk + hk * Dk, L * sk * 2);
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int e = u + 256 * q4;
      st.k[q4] = buf_ld16(kr, uint32_t((e >> 4) * sk + (e & 15) * 8) * 2);
    }
    const auto tr = buffer_rsrc(tl->t[0], 2 * kTri * 2);
#pragma unroll
    for (int t = 0; t < 3; ++t) st.tb[t] = buf_ld16(tr, uint32_t(u + 256 * t) * 16);
  };
  auto load2 = [&](Stage& st, int c) {
    const int64_t slot = sq.slot0 + c, tok = sq.tok0 + int64_t(c) * kC;
    const uint32_t L = uint32_t(min(kC, sq.len - c * kC));
    const Tile* tl = a.tiles + (slot * a.Hv + hv);
    const auto qr = buffer_rsrc(a.q + tok * sk + hk * Dk, L * sk * 2);
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int e = u + 256 * q4;
      st.q[q4] = buf_ld16(qr, uint32_t((e >> 4) * sk + (e & 15) * 8) * 2);
    }
    const auto gr = buffer_rsrc(tl->gam, 3 * kC * 4);  // gam, dec, beta
    st.gd = buf_ld4(gr, uint32_t(u) * 4);
    const auto vr = buffer_rsrc(a.v + tok * sv + hv * a.Dv + row0, L * sv * 2);
    st.v = buf_ld16(vr, u < 8 * kRows ? uint32_t((u / (kRows / 8)) * sv + 8 * (u % (kRows / 8))) * 2 : 0x80000000u);
    const auto pr = buffer_rsrc(tl->p[0], 2 * kTri * 2);  // hi, then lo
#pragma unroll
    for (int t = 0; t < 3; ++t) st.p[t] = buf_ld16(pr, uint32_t(u + 256 * t) * 16);
  };
  // k and packed T, then v, the per-position vectors and q: to buffer b of the chain and to Qb.
  auto stage1 = [&](const Stage& st, int b) {
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int e = u + 256 * q4;
      *reinterpret_cast<uint4*>(Kb[b] + swz(e >> 4, (e & 15) * 8, kLK)) = st.k[q4];
    }
#pragma unroll
    for (int t = 0; t < 2; ++t) *reinterpret_cast<uint4*>(Tbp[b] + 8 * (u + 256 * t)) = st.tb[t];
    if (w < 10) *reinterpret_cast<uint4*>(Tbp[b] + 8 * (u + 512)) = st.tb[2];  // units 640.. are padding
  };
  auto stage2 = [&](const Stage& st, int b) {
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int e = u + 256 * q4;
      *reinterpret_cast<uint4*>(Qb + swz(e >> 4, (e & 15) * 8, kLK)) = st.q[q4];
    }
    if (w < 11) Gs[b][u] = st.gd;                                                 // units 192.. are padding
    if (kRows == 32 || w < 10) *reinterpret_cast<uint4*>(Vs[b] + 8 * u) = st.v;  // 16 rows: units 128.. padding
  };
  auto stage_p = [&](const Stage& st) {
#pragma unroll
    for (int t = 0; t < 2; ++t) *reinterpret_cast<uint4*>(Pb + 8 * (u + 256 * t)) = st.p[t];
    if (w < 10) *reinterpret_cast<uint4*>(Pb + 8 * (u + 512)) = st.p[2];
  };

  // Each group runs a loop of its own with the chain's three barriers per chunk (a barrier counts waves, not program
  // points): each loop then holds only its own group's memory operations, and the compiler's waits in it are exact.
  if (w >= 8) {
    // Two register sets take turns, cur holding chunk c (staged but for its P) and nxt chunk c + 1, and the LDS
    // writes go where the chain's phases leave the LDS least busy. After the chain's first barrier of chunk c:
    // chunk c + 1's k and T to the chain's other LDS buffers (their last readers were chunk c - 1's), and the first
    // part of chunk c + 2 into cur (two chunks ahead, which covers the memory latency). After the second: chunk c's
    // P to Pb (chunk c - 1's y is formed) and the second part of chunk c + 2. After the third: chunk c + 1's q to Qb
    // (chunk c's S Q^T is done), its v and per-position vectors.
    auto step = [&](int c, Stage& cur, Stage& nxt) {
      const int c2 = min(c + 2, nch - 1);  // the last chunks load the last again rather than branch
      const int b1 = (c & 1) ^ 1;
      __syncthreads();
      load1(cur, c2);
      stage1(nxt, b1);
      __syncthreads();
      stage_p(cur);
      load2(cur, c2);
      __syncthreads();
      stage2(nxt, b1);
    };
    Stage sa, sb;
    if (nch > 0) {
      const int c1 = min(1, nch - 1);
      load1(sa, 0);
      load2(sa, 0);
      load1(sb, c1);
      load2(sb, c1);
      stage1(sa, 0);
      stage2(sa, 0);
    }
    int c = 0;
    for (; c + 1 < nch; c += 2) {
      step(c, sa, sb);
      step(c + 1, sb, sa);
    }
    if (c < nch) step(c, sa, sb);
    return;
  }
  if (w >= 4) {
    for (int c = 0; c < nch; ++c) {
      const int b = c & 1;
      __syncthreads();
      // S K^T and S Q^T at state rows 16 rt + 4g + jj, position ip, from one read of S (hi and lo) per row tile;
      // then R^T = (V^T - (S K^T) diag(exp G)) diag(beta), which the chain's next phase reads.
      f32x4 kh[kRT], kl[kRT], xh[kRT], xl[kRT];
#pragma unroll
      for (int rt = 0; rt < kRT; ++rt) kh[rt] = zero4(), kl[rt] = zero4(), xh[rt] = zero4(), xl[rt] = zero4();
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const int ak = swz(ip, 32 * s + 8 * g, kLK);
        const bf16x8 bk = lds8(Kb[b] + ak), bq = lds8(Qb + ak);
#pragma unroll
        for (int rt = 0; rt < kRT; ++rt) {
          const int at = swz(16 * rt + li, 32 * s + 8 * g, kLS);
          const bf16x8 sh = lds8(Sm[0] + at), sl = lds8(Sm[1] + at);
          kh[rt] = mma(kh[rt], sh, bk);
          kl[rt] = mma(kl[rt], sl, bk);
          xh[rt] = mma(xh[rt], sh, bq);
          xl[rt] = mma(xl[rt], sl, bq);
        }
      }
      const float gam = Gs[b][ip];
      {
        const float bet = Gs[b][2 * kC + ip];
#pragma unroll
        for (int rt = 0; rt < kRT; ++rt) {
          const uint2 v = *reinterpret_cast<const uint2*>(Vs[b] + kRows * ip + 16 * rt + 4 * g);
          const f32x4 ks = kh[rt] + kl[rt];
          const f32x4 r = {bf16_lo(v.x) - gam * ks[0], bf16_hi(v.x) - gam * ks[1], bf16_lo(v.y) - gam * ks[2],
                           bf16_hi(v.y) - gam * ks[3]};
          put4(Wm[0], Wm[1], swz(ip, oR + 16 * rt + 4 * g, kLP), bet * r);
        }
      }
      f32x4 xs[kRT];
#pragma unroll
      for (int rt = 0; rt < kRT; ++rt) xs[rt] = xh[rt] + xl[rt];
      __syncthreads();
      __syncthreads();
      // Y^T = (S Q^T) diag(exp G) + Delta^T P^T at state rows 16 rt + 4g + jj, position ip; P rows ip from the packed
      // copy (blocks above the diagonal are zeros).
      const int64_t tok = sq.tok0 + int64_t(c) * kC;
      const uint32_t L = uint32_t(min(kC, sq.len - c * kC));
      // Positions past the chunk's end fall past the resource and are dropped.
      const auto yr = buffer_rsrc(y + tok * sv + hv * a.Dv + row0, L * sv * uint32_t(sizeof(OutT)));
      Split8 PB[2];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int c8 = 32 * s + 8 * g;
        const bool in = (c8 >> 4) <= wp;
        const int at = in ? tri_off(ip, c8) : 0;
        const bf16x8 z = {};
        const bf16x8 ph = lds8(Pb + at), pl = lds8(Pb + kTri + at);
        PB[s] = Split8{in ? ph : z, in ? pl : z};
      }
#pragma unroll
      for (int rt = 0; rt < kRT; ++rt) {
        f32x4 yv = gam * xs[rt];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const __bf16* D0 = Wm[0] + 32 * s * kLP + oD + 16 * rt;
          const __bf16* D1 = Wm[1] + 32 * s * kLP + oD + 16 * rt;
          yv = mma3(yv, Split8{lds_tr8s(D0, kLP, lane), lds_tr8s(D1, kLP, lane)}, PB[s]);
        }
        BufIO<OutT>::st4(yr, uint32_t(ip * sv + 16 * rt + 4 * g), yv);
      }
    }
    return;
  }

  // Waves 0-3. State: tile (rt, t) holds S[16 rt + li][32 wp + 16 t + 4 g + jj]. (s0 and s_out need only 4-byte
  // alignment: one element at a time.)
  f32x4 S[kRT][2];
#pragma unroll
  for (int rt = 0; rt < kRT; ++rt) S[rt][0] = zero4(), S[rt][1] = zero4();
  if (a.s0) {
#pragma unroll
    for (int rt = 0; rt < kRT; ++rt)
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) S[rt][t][jj] = a.s0[(srow + 16 * rt) * Dk + 32 * wp + 16 * t + 4 * g + jj];
  }
  const uint32_t ck_bytes = a.ckpt ? uint32_t(kRows) * Dk * 4 : 0u;  // a forward without checkpoints drops the stores
  for (int c = 0; c < nch; ++c) {
    const int64_t slot = sq.slot0 + c;
    const int b = c & 1;
    {  // S to LDS, split, and to the checkpoint (the last readers of Sm are two barriers back)
      const float* ckb = a.ckpt ? a.ckpt + ((slot * a.Hv + hv) * a.Dv + row0) * Dk : a.s0;
      const auto ck = buffer_rsrc(ckb, ck_bytes);
#pragma unroll
      for (int rt = 0; rt < kRT; ++rt)
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int col = 32 * wp + 16 * t + 4 * g;
          put4(Sm[0], Sm[1], swz(16 * rt + li, col, kLS), S[rt][t]);
          BufIO<float>::st4(ck, uint32_t((16 * rt + li) * Dk + col), S[rt][t]);
        }
    }
    __syncthreads();  // S in LDS: the output group forms R from it
    __syncthreads();  // R in LDS

    // Delta^T = R^T T^T (R with beta applied): A = R^T through the transposing read, B = T rows ip from the packed
    // copy.
    {
      Split8 TB[2];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int c8 = 32 * s + 8 * g;
        const bool in = (c8 >> 4) <= wp;  // blocks above the diagonal are zeros
        const int at = in ? tri_off(ip, c8) : 0;
        const bf16x8 z = {};
        const bf16x8 th = lds8(Tbp[b] + at), tl = lds8(Tbp[b] + kTri + at);
        TB[s] = Split8{in ? th : z, in ? tl : z};
      }
      const float dec = Gs[b][kC + ip];
#pragma unroll
      for (int rt = 0; rt < kRT; ++rt) {
        f32x4 d2[2];  // the two k steps in independent chains
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const __bf16* R0 = Wm[0] + 32 * s * kLP + oR + 16 * rt;
          const __bf16* R1 = Wm[1] + 32 * s * kLP + oR + 16 * rt;
          d2[s] = mma3(zero4(), Split8{lds_tr8s(R0, kLP, lane), lds_tr8s(R1, kLP, lane)}, TB[s]);
        }
        const f32x4 dl = d2[0] + d2[1];
        put4(Wm[0], Wm[1], swz(ip, oD + 16 * rt + 4 * g, kLP), dl);
        put4(Wm[0], Wm[1], swz(ip, oDD + 16 * rt + 4 * g, kLP), dec * dl);
      }
    }
    __syncthreads();

    // S^T <- exp(G_63) S^T + K^T (D Delta): A = K^T rows 32 wp + 16 t + li and B = D Delta, both through the
    // transposing read.
    const float glast = Gs[b][kC - 1];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      bf16x8 KA[2];
#pragma unroll
      for (int t = 0; t < 2; ++t) KA[t] = lds_tr8s(Kb[b] + swz(32 * s, 32 * wp + 16 * t, kLK), kLK, lane);
#pragma unroll
      for (int rt = 0; rt < kRT; ++rt) {
        const __bf16* E0 = Wm[0] + 32 * s * kLP + oDD + 16 * rt;
        const __bf16* E1 = Wm[1] + 32 * s * kLP + oDD + 16 * rt;
        const Split8 B{lds_tr8s(E0, kLP, lane), lds_tr8s(E1, kLP, lane)};
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          if (s == 0) S[rt][t] = glast * S[rt][t];
          S[rt][t] = mma2(S[rt][t], KA[t], B);
        }
      }
    }
  }
  if (a.s_out) {
#pragma unroll
    for (int rt = 0; rt < kRT; ++rt)
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) a.s_out[(srow + 16 * rt) * Dk + 32 * wp + 16 * t + 4 * g + jj] = S[rt][t][jj];
  }
}

}  // namespace

hipError_t launch_chunk_fwd(const ChunkArgs& a, bool out_bf16, hipStream_t s) {
  const int total = a.nblk * a.Hv * a.N;
  const bool r32 = a.Dv == 32 * a.nblk;  // 32 state rows per block (else 16)
  void (*k)(ChunkArgs) = out_bf16 ? (r32 ? chunk_fwd_kernel<bf16_t, 32> : chunk_fwd_kernel<bf16_t, 16>)
                                  : (r32 ? chunk_fwd_kernel<float, 32> : chunk_fwd_kernel<float, 16>);
  hipLaunchKernelGGL(k, dim3(total), dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace qbgdn
