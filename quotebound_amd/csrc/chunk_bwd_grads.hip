// Chunked design, kernel 4: the per-chunk gradients. One work item (8 waves) per (chunk slot, key head); the value
// heads of the key head's GQA group run in order and their dq, dk contributions add up in registers, so the sums
// over value heads have a fixed order (reference src/delta_grad.cpp:194-198) and need no atomics. The grid is one
// resident block per CU looping over items, so the next item's first value head is read during this item's last
// end phase, as a value head's is during the previous head's.
//
// Per value head, with S0 the chunk's start state (checkpoint), dS its end-state cotangent (from the backward state
// pass) and the chunk's tile (T, P, exp G, D, beta from prep), the state rows are streamed in blocks of 32:
//   KS = K S0^T, R = V - diag(exp G) KS, Delta = T (diag(beta) R), KdS = K dS^T,
//   dDelta = P^T dY + D KdS, dR' = T^T dDelta, dR = diag(beta) dR'     (D = diag(exp(G_63 - G)))
//   dP^T += Delta dY^T, dT^T += (diag(beta) R) dDelta^T, dbeta += rowsum(R * dR'),
//   dQ_inter += dY S0, dK += -diag(exp G) dR S0 + D Delta dS
// then, once per value head, the 64 x 64 part:
//   dQ += diag(exp G) dQ_inter + (dP * M) K,  dK += (dP * M)^T Q + (dKK + dKK^T) K
//   dA = -T^T dT T^T,  dKK = strict_lower(diag(beta) dA * E)
//   dbeta_j += sum_m dA_jm E_jm (K K^T)_jm,  dG from every exp(.) factor, dg = reverse cumsum
// (dbeta's first term, sum_i dTb_ij T_ij with Tb = T diag(beta), equals sum_r R_jr (T^T dDelta)_jr.)
// (tests/chunk_math.py restates these equations and checks them against the oracle.) Wave w owns positions
// 16 (w % 4) .. + 15 and, within each product, the half w / 4 of the other index (state rows of a 32-row block,
// key-position tiles, or 64 of the 128 columns). MFMA with split float32 operands as in the forward. Each
// intermediate crosses between waves through LDS once, written as 8-byte vectors and read either directly or with
// gfx950's transposing LDS read, whichever index the consuming product reduces over.
// Sums reduced over a lane group (sum16 and the lane-swap sums give every lane of the group the same bits) are
// stored by every lane of the group: a store under a lane-0 condition would be an exec-masked branch.
#include <type_traits>

#include "chunk_common.h"
#include "chunk_kernels.h"
#include "prologue_math.h"

namespace qbgdn {
namespace {

constexpr int kThreads = 512;
// Block-loop region (bf16 element offsets), one 32-row block of the state at a time. Every matrix is stored once, as
// hi and lo halves: S0, dS as rows [r][c]; dY as rows [i][r]; the per-position results as [r][i]. Products that
// reduce over the contiguous index read 16 bytes per lane; those that reduce over the other index use the
// transposing read (lds_tr8). The row strides put the four rows each transposing read touches, and the eight rows
// each 16-byte read touches, on distinct banks.
constexpr int kLS = 144;  // S0, dS [32][128]
constexpr int kLY = 48;   // dY [64][32]
constexpr int kLP = 80;   // [32][64]
constexpr int kLT = 80;   // T, P [64][64]
constexpr int oS0h = 0, oS0l = oS0h + 32 * kLS, odSh = oS0l + 32 * kLS, odSl = odSh + 32 * kLS;
constexpr int odYh = odSl + 32 * kLS, odYl = odYh + kC * kLY;
constexpr int oRh = odYl + kC * kLY, oRl = oRh + 32 * kLP;        // diag(beta) R, R = V - diag(exp G) K S0^T
constexpr int oDh = oRl + 32 * kLP, oDl = oDh + 32 * kLP;         // Delta
constexpr int oDDh = oDl + 32 * kLP, oDDl = oDDh + 32 * kLP;      // D Delta
constexpr int odDh = oDDl + 32 * kLP, odDl = odDh + 32 * kLP;     // dDelta
constexpr int oGdRh = odDl + 32 * kLP, oGdRl = oGdRh + 32 * kLP;  // -diag(exp G) dR
constexpr int kLoopBytes = (oGdRl + 32 * kLP) * 2;
// End-phase region (aliases the block-loop region), bf16 element offsets: Q rows, then P * M, Z^T (Z = dT T^T) and
// dKK^T, each as hi and lo 64 x 64 matrices; then float32 per-position partial sums. (K rows stay in their own array
// for the whole block and T in TL for the whole value head; dT reuses the P array.)
constexpr int kLK = 144;
constexpr int eQb = 0;
constexpr int eMh = eQb + kC * kLK, eMl = eMh + kC * kLT;  // P * M
constexpr int eZh = eMl + kC * kLT, eZl = eZh + kC * kLT;
constexpr int eKh = eZl + kC * kLT, eKl = eKh + kC * kLT;
constexpr int eF = (eKl + kC * kLT) / 2;  // first float32 offset
constexpr int eX2r = eF, eX2c = eX2r + 2 * kC, edbA = eX2c + 4 * kC;
constexpr int ex1c = edbA + 2 * kC, etq = ex1c + 4 * kC;
constexpr int kEndBytes = (etq + 2 * kC) * 4;
constexpr int kSmemBytes = kLoopBytes > kEndBytes ? kLoopBytes : kEndBytes;

// The key tile (16 positions j) that accumulator mi of the wave at position tile pw, half hw holds in dP^T and
// dT^T. Only tiles m <= pw carry work. For each pw the two halves together hold all four tiles; positions 0..31
// alternate the tiles between halves so each half works on one of the tiles 0..pw, positions 32..63 split them in
// halves. The busiest wave of the phase that accumulates them then runs 5 products in place of 6.
__device__ __forceinline__ int key_tile(int pw, int hw, int mi) { return pw < 2 ? hw + 2 * mi : 2 * hw + mi; }

// kFused: the layer's prologue backward at the end (qb_gdn_bwd_prologue; bf16 only). The cotangents of q, k and
// beta are rounded to bf16 as the separate pass would read them, then turned into those of q_raw, k_raw, a and b with
// the separate pass's arithmetic (prologue_math.h); the dA_log and ddt_bias terms are summed per (chunk, value head)
// into a.pro.part, which chunk_gate_sums_kernel sums over chunks.
// kSplit: short sequences, a.dqk_part set (a separate instantiation, so that the long-sequence kernel carries none of
// its indexing).
template <typename OutT, bool kFused, bool kSplit>
__global__ __launch_bounds__(kThreads) void chunk_bwd_grads_kernel(ChunkArgs a) {
  constexpr int Dk = 128;
  constexpr bool kExactDy = std::is_same<OutT, bf16_t>::value;
  __shared__ __align__(16) unsigned char smem[kSmemBytes];
  __shared__ __align__(16) __bf16 Kres[kC * kLK];  // the chunk's K rows, for the whole block
  // The value head's T and P (bf16 hi and lo, rows i, columns j), staged once per head: A operands of T rows
  // directly, of T^T and P^T rows through the transposing read.
  __shared__ __align__(16) __bf16 TL[2][kC * kLT], PL[2][kC * kLT];
  __shared__ float gam[kC], dec[kC], bet[kC], Gf[kC];
  __shared__ float gpos[2][kC], hpos[2][kC], bpos[2][kC], red[kThreads / 64];
  __bf16* sb = reinterpret_cast<__bf16*>(smem);
  float* sf = reinterpret_cast<float*>(smem);
  typedef float Row[kC];
  Row* x2r = reinterpret_cast<Row*>(sf + eX2r);
  Row* x2c = reinterpret_cast<Row*>(sf + eX2c);
  Row* dbAp = reinterpret_cast<Row*>(sf + edbA);
  Row* x1cp = reinterpret_cast<Row*>(sf + ex1c);
  Row* tpos = reinterpret_cast<Row*>(sf + etq);

  // kSplit: one work item per (chunk slot, key head, value head), whose dq and dk go to the partials for
  // chunk_dqk_sum_kernel; otherwise one per (chunk slot, key head), the group's value heads in turn.
  const int grp = a.Hv / a.Hk, hs = kSplit ? grp : 1, total = int(a.lay.NC) * a.Hk * hs;
  // Lane roles (position tile pw = w % 4, half hw = w / 4, lane group g, lane li) are derived where they are used, from
  // an opaque copy of the thread index, so that their address expressions are not held across the loops.
  const int tid = threadIdx.x;
  const OutT* dy = static_cast<const OutT*>(a.dy);
  const int sk = a.Hk * Dk, sv = a.Hv * a.Dv;  // token strides of k/q/dq/dk and v/dy
  // A work item: a chunk slot, key head and its value heads [e0, e0 + ne). The grid is persistent: block b takes items
  // b, b + gridDim.x, ..., and gridDim.x is a multiple of 8, so all of a block's items fall in its own XCD's range of
  // xcd_remap.
  struct Item {
    int64_t slot, tok;
    int hk, L, e0, ne;
  };
  auto item_at = [&](int id) {
    const int wid = xcd_remap(id, total);
    const int64_t slot = wid / (a.Hk * hs);
    const int rem = wid % (a.Hk * hs);
    const SlotPos sp = slot_pos(a.tab, slot);
    return Item{slot, sp.tok, rem / hs, sp.L, kSplit ? rem % hs : 0, kSplit ? 1 : grp};
  };

  // Global reads, kept in registers from issue to staging. A value head's tile (T and P rows hi and lo, thread ->
  // row lt / 8, columns 8 (lt % 8) .. + 7, zeros above the diagonal blocks; and the per-position scalars, thread lt <
  // 64) and one 32-row block of its state (S0 and dS rows, dY, v). dy and v go through buffer resources that end at
  // the chunk's last row, so rows past it read as zeros without a branch.
  struct TileIn {
    bf16x8 tp[4];  // T hi, T lo, P hi, P lo
    float sc[4];   // exp G, exp(G_63 - G), beta, G
  };
  struct BlockIn {
    float4 xs[2], ys[2];  // S0, dS: thread -> row tid / 16, columns 8 (tid % 16) .. + 7
    uint4 yraw;           // dY: thread -> position tid / 8, rows 4 (tid % 8) .. + 3
    uint16_t vraw[4];     // v at the wave's accumulator positions (16 pw + 4g + jj, column 16 hw + li)
  };
  auto load_tile = [&](TileIn& ti, const Item& it, int hv, int lt) {
    const Tile* tl = a.tiles + it.slot * a.Hv + hv;
    if (lt < kC) ti.sc[0] = tl->gam[lt], ti.sc[1] = tl->dec[lt], ti.sc[2] = tl->beta[lt], ti.sc[3] = tl->G[lt];
    const auto tr = buffer_rsrc(tl->t[0], 4 * kTri * 2);  // t[0], t[1], p[0], p[1] are contiguous
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) ti.tp[q4] = tri_ld8(tr, q4 * kTri, lt >> 3, (lt & 7) * 8);
  };
  auto load_rows = [&](float4 (&x)[2], const float* base, const Item& it, int hv, int r0, int lt) {
    const float* p = base + ((it.slot * a.Hv + hv) * a.Dv + r0) * Dk + (lt >> 4) * Dk + (lt & 15) * 8;
    x[0] = *reinterpret_cast<const float4*>(p);
    x[1] = *reinterpret_cast<const float4*>(p + 4);
  };
  auto load_dy_v = [&](BlockIn& b, const Item& it, int hv, int r0, int lt) {
    const int g = (lt >> 4) & 3, li = lt & 15, pw = (lt >> 6) & 3, hw = lt >> 8;
    const auto yr = buffer_rsrc(dy + (it.tok * a.Hv + hv) * a.Dv + r0, uint32_t(it.L * sv) * uint32_t(sizeof(OutT)));
    const auto vr = buffer_rsrc(a.v + (it.tok * a.Hv + hv) * a.Dv + r0, uint32_t(it.L * sv) * 2u);
    const int iy = lt >> 3, r4 = (lt & 7) * 4;
    if constexpr (kExactDy) {
      const auto t2 = __builtin_amdgcn_raw_buffer_load_b64(yr, int(uint32_t(iy * sv + r4) * 2), 0, 0);
      b.yraw = uint4{t2[0], t2[1], 0u, 0u};
    } else {
      b.yraw = buf_ld16(yr, uint32_t(iy * sv + r4) * 4);
    }
#pragma unroll
    for (int jj = 0; jj < 4; ++jj)
      b.vraw[jj] = buf_ld2(vr, uint32_t((16 * pw + 4 * g + jj) * sv + 16 * hw + li) * 2);
  };
  // A value head's tile and first block, issued one value head ahead (the block's first head here at the start, the
  // others in pieces during the previous head's end phase, the next item's first head during this item's last end
  // phase), so no head waits on a global read before its first block.
  auto load_head = [&](TileIn& ti, BlockIn& b, const Item& it, int hv) {
    int lt = tid;
    asm volatile("" : "+v"(lt));
    load_tile(ti, it, hv, lt);
    load_rows(b.xs, a.ckpt, it, hv, 0, lt);
    load_rows(b.ys, a.dsend, it, hv, 0, lt);
    load_dy_v(b, it, hv, 0, lt);
  };
  TileIn ti;
  BlockIn nb;
  {
    const Item first = item_at(blockIdx.x);
    load_head(ti, nb, first, first.hk * grp + first.e0);
  }
  for (int id = blockIdx.x; id < total; id += gridDim.x) {
    const Item cur = item_at(id);
    const int64_t slot = cur.slot, tok = cur.tok;
    const int hk = cur.hk, L = cur.L;
    const bf16_t* kbase = a.k + tok * sk + hk * Dk;
    const bf16_t* qbase = a.q + tok * sk + hk * Dk;
    // Rows past the chunk's last row read as zeros.
    const auto krs = buffer_rsrc(kbase, uint32_t(L * sk) * 2u), qrs = buffer_rsrc(qbase, uint32_t(L * sk) * 2u);
    __syncthreads();  // the previous item's readers of the K rows and the per-position arrays are done

    // The chunk's K rows (A operands of K S0^T, K dS^T, K K^T; B of the K products of the end phase).
    for (int e = tid; e < kC * 16; e += kThreads) {
      const int t = e >> 4, c8 = (e & 15) * 8;
      *reinterpret_cast<uint4*>(Kres + swz(t, c8, kLK)) = buf_ld16(krs, uint32_t(t * sk + c8) * 2);
    }
    f32x4 dQ[4], dK[4];  // columns 16 (4 hw + t) + li, rows 16 pw + 4 g + jj
#pragma unroll
    for (int t = 0; t < 4; ++t) dQ[t] = zero4(), dK[t] = zero4();
    // (K K^T)[p][m], rows p = 16 pw + 4g + jj, columns m = 16 key_tile(pw, hw, mi) + li; zero above tile pw. The same
    // for every value head of the group: formed in the item's first one's end phase.
    f32x4 kk[2];

    for (int e = cur.e0; e < cur.e0 + cur.ne; ++e) {
      const int hv = hk * grp + e;
      // The head whose tile and first block the end phase reads ahead, in pieces at the starts of E2, E3 and E4
      // (beside their products, so that no phase issues them all): the next in the group, the next item's first,
      // or, for the block's last item, this head again (those reads are unused; they keep every path's loads the
      // same, so the compiler's waits stay exact).
      Item nx = cur;
      int nhv = hv;
      if (e + 1 < cur.e0 + cur.ne) {
        nhv = hv + 1;
      } else if (id + int(gridDim.x) < total) {
        nx = item_at(id + gridDim.x);
        nhv = nx.hk * grp + nx.e0;
      }
      __syncthreads();
      if (tid < kC) gam[tid] = ti.sc[0], dec[tid] = ti.sc[1], bet[tid] = ti.sc[2], Gf[tid] = ti.sc[3];
      {  // T and P, hi and lo
        const int lt8 = swz(tid >> 3, (tid & 7) * 8, kLT);
        *reinterpret_cast<bf16x8*>(TL[0] + lt8) = ti.tp[0];
        *reinterpret_cast<bf16x8*>(TL[1] + lt8) = ti.tp[1];
        *reinterpret_cast<bf16x8*>(PL[0] + lt8) = ti.tp[2];
        *reinterpret_cast<bf16x8*>(PL[1] + lt8) = ti.tp[3];
      }
      f32x4 dPt[2], dTt[2], dQi[4];  // dPt, dTt: key tiles m = key_tile(pw, hw, mi); lane -> column i = ip, rows j
#pragma unroll
      for (int t = 0; t < 2; ++t) dPt[t] = zero4(), dTt[t] = zero4();
#pragma unroll
      for (int t = 0; t < 4; ++t) dQi[t] = zero4();
      float gpart[4] = {0.f, 0.f, 0.f, 0.f}, hD[4] = {0.f, 0.f, 0.f, 0.f}, bpart[4] = {0.f, 0.f, 0.f, 0.f}, sds = 0.f;
      __syncthreads();

      // The end phase's inputs (Q rows, as bf16 bits), loaded during the value head's last block into the registers
      // the next block's reads would use: thread -> Q row e / 16, columns 8 (e % 16) .. + 7 for e = tid, tid + 512.
      auto load_end = [&](BlockIn& b, int lt) {
#pragma unroll
        for (int q2 = 0; q2 < 2; ++q2) {
          const int e = lt + kThreads * q2, t = e >> 4, c8 = (e & 15) * 8;
          b.ys[q2] = __builtin_bit_cast(float4, buf_ld16(qrs, uint32_t(t * sk + c8) * 2));
        }
      };

      // One 32-row block of the state. The last block of the value head (more = false) loads the end phase's inputs
      // instead of the next block's: it is a separate copy of the code, so that every copy issues the same loads in
      // the same order whatever the path, and the compiler's count of outstanding loads stays exact.
      auto block = [&](const int r0, auto more_tag) {
        constexpr bool more = decltype(more_tag)::value;
        // Lane indices re-derived from an opaque copy, so their many address expressions are recomputed here instead
        // of being hoisted out of both loops and held (spilled) for the whole kernel.
        int lt = tid;
        asm volatile("" : "+v"(lt));
        const int g = (lt >> 4) & 3, li = lt & 15, pw = (lt >> 6) & 3, hw = lt >> 8, ip = 16 * pw + li;
        const int sr = lt >> 4, sc = (lt & 15) * 8, iy = lt >> 3, r4 = (lt & 7) * 4;
        const float4* xs = nb.xs;
        const float4* ys = nb.ys;
        const uint4 yraw = nb.yraw;
        __syncthreads();  // the previous block's readers of LDS are done

        {  // Stage S0, dS rows and dY rows as hi / lo.
          const float x[8] = {xs[0].x, xs[0].y, xs[0].z, xs[0].w, xs[1].x, xs[1].y, xs[1].z, xs[1].w};
          const float y[8] = {ys[0].x, ys[0].y, ys[0].z, ys[0].w, ys[1].x, ys[1].y, ys[1].z, ys[1].w};
#pragma unroll
          for (int u = 0; u < 8; ++u) sds += x[u] * y[u];
          const Split8 xsp = split8(x), ysp = split8(y);
          const int at = swz(sr, sc, kLS);
          *reinterpret_cast<bf16x8*>(sb + oS0h + at) = xsp.hi;
          *reinterpret_cast<bf16x8*>(sb + oS0l + at) = xsp.lo;
          *reinterpret_cast<bf16x8*>(sb + odSh + at) = ysp.hi;
          *reinterpret_cast<bf16x8*>(sb + odSl + at) = ysp.lo;
          if constexpr (kExactDy) {
            *reinterpret_cast<uint2*>(sb + odYh + swz(iy, r4, kLY)) = uint2{yraw.x, yraw.y};
          } else {
            put4(sb + odYh, sb + odYl, swz(iy, r4, kLY), __uint_as_float(yraw.x), __uint_as_float(yraw.y),
                 __uint_as_float(yraw.z), __uint_as_float(yraw.w));
          }
        }
        float vv[4];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) vv[jj] = bf16_to_f32(nb.vraw[jj]);
        __syncthreads();
        if constexpr (more)
          load_rows(nb.xs, a.ckpt, cur, hv, r0 + 32, lt);  // the next block's reads, first group
        else
          load_end(nb, lt);

        // The wave's own dY rows (i = ip, k = r = 8g..): A of dY S0, B of Delta dY^T.
        Split8 dYo;
        dYo.hi = lds8(sb + odYh + swz(ip, 8 * g, kLY));
        if constexpr (!kExactDy) dYo.lo = lds8(sb + odYl + swz(ip, 8 * g, kLY));

        // Phase 1: KS and KdS for positions i = 16 pw + 4g + jj, state rows r = 16 hw + li.
        const int r = 16 * hw + li, i0 = 16 * pw + 4 * g;
        f32x4 ks = zero4(), kds = zero4();
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int at = swz(r, 32 * s + 8 * g, kLS);
          const bf16x8 ka = lds8(Kres + swz(ip, 32 * s + 8 * g, kLK));
          ks = mma(mma(ks, ka, lds8(sb + oS0h + at)), ka, lds8(sb + oS0l + at));
          kds = mma(mma(kds, ka, lds8(sb + odSh + at)), ka, lds8(sb + odSl + at));
        }
        float gks[4], rv[4];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          gks[jj] = gam[i0 + jj] * ks[jj];
          rv[jj] = vv[jj] - gks[jj];
        }
        put4(sb + oRh, sb + oRl, swz(r, i0, kLP), bet[i0] * rv[0], bet[i0 + 1] * rv[1], bet[i0 + 2] * rv[2],
             bet[i0 + 3] * rv[3]);
        __syncthreads();
        if constexpr (more) load_rows(nb.ys, a.dsend, cur, hv, r0 + 32, lt);

        // Phase 2: Delta = T (diag(beta) R) and dDelta = P^T dY + D KdS (rows: the wave's positions; lane: row r).
        f32x4 dl = zero4(), dd;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          if (s == 0 || pw >= 2) {  // T is zero above the diagonal blocks: rows 0..31 end at column 31
            const int at = swz(r, 32 * s + 8 * g, kLP), atb = swz(ip, 32 * s + 8 * g, kLT);
            const Split8 TA{lds8(TL[0] + atb), lds8(TL[1] + atb)};
            dl = mma3(dl, TA, Split8{lds8(sb + oRh + at), lds8(sb + oRl + at)});
          }
        }
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) dd[jj] = dec[i0 + jj] * kds[jj];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          if (32 * s + 31 >= 16 * pw) {  // P^T is zero below the diagonal
            const int at = 32 * s * kLY + 16 * hw;
            // P^T rows ip (k = i): P's rows 32s.., column ip.
            const Split8 PA{lds_tr8s(PL[0] + 32 * s * kLT + 16 * pw, kLT, lt), lds_tr8s(PL[1] + 32 * s * kLT + 16 * pw, kLT, lt)};
            if constexpr (kExactDy)
              dd = mma2(dd, PA, lds_tr8s(sb + odYh + at, kLY, lt));
            else
              dd = mma3(dd, PA, Split8{lds_tr8s(sb + odYh + at, kLY, lt), lds_tr8s(sb + odYl + at, kLY, lt)});
          }
        }
        {
          float ddl[4];
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            hD[jj] += dec[i0 + jj] * dl[jj] * kds[jj];
            ddl[jj] = dec[i0 + jj] * dl[jj];
          }
          put4(sb + oDh, sb + oDl, swz(r, i0, kLP), dl[0], dl[1], dl[2], dl[3]);
          put4(sb + oDDh, sb + oDDl, swz(r, i0, kLP), ddl[0], ddl[1], ddl[2], ddl[3]);
          put4(sb + odDh, sb + odDl, swz(r, i0, kLP), dd[0], dd[1], dd[2], dd[3]);
        }
        __syncthreads();
        if constexpr (more) load_dy_v(nb, cur, hv, r0 + 32, lt);

        // Phase 3: dR = diag(beta) T^T dDelta (and dbeta's T part, R * (T^T dDelta) summed over the rows); dP^T +=
        // Delta dY^T and dT^T += (diag(beta) R) dDelta^T over this half's key tiles.
        {
          f32x4 dr = zero4();
#pragma unroll
          for (int s = 0; s < 2; ++s) {
            if (32 * s + 31 >= 16 * pw) {  // T^T is zero below the diagonal
              const int at = swz(r, 32 * s + 8 * g, kLP);
              // T^T rows ip (k = j): T's rows 32s.., column ip.
              const Split8 TtA{lds_tr8s(TL[0] + 32 * s * kLT + 16 * pw, kLT, lt),
                               lds_tr8s(TL[1] + 32 * s * kLT + 16 * pw, kLT, lt)};
              dr = mma3(dr, TtA, Split8{lds8(sb + odDh + at), lds8(sb + odDl + at)});
            }
          }
          float gdr[4];
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            bpart[jj] += rv[jj] * dr[jj];
            dr[jj] *= bet[i0 + jj];
            gpart[jj] -= dr[jj] * gks[jj];
            gdr[jj] = -gam[i0 + jj] * dr[jj];
          }
          put4(sb + oGdRh, sb + oGdRl, swz(r, i0, kLP), gdr[0], gdr[1], gdr[2], gdr[3]);
        }
        {
          // dDelta[i][r] of the wave's positions as B (k = r, n = i).
          const Split8 BdD{lds_tr8s(sb + odDh + 16 * pw, kLP, lt), lds_tr8s(sb + odDl + 16 * pw, kLP, lt)};
#pragma unroll
          for (int mi = 0; mi < 2; ++mi) {
            const int m = key_tile(pw, hw, mi);
            if (m <= pw) {
              // Delta and diag(beta) R rows j of key tile m as A (m = j, k = r).
              const Split8 AD{lds_tr8s(sb + oDh + 16 * m, kLP, lt), lds_tr8s(sb + oDl + 16 * m, kLP, lt)};
              if constexpr (kExactDy)
                dPt[mi] = mma2(dPt[mi], AD, dYo.hi);
              else
                dPt[mi] = mma3(dPt[mi], AD, dYo);
              const Split8 AR{lds_tr8s(sb + oRh + 16 * m, kLP, lt), lds_tr8s(sb + oRl + 16 * m, kLP, lt)};
              dTt[mi] = mma3(dTt[mi], AR, BdD);
            }
          }
        }
        __syncthreads();

        // Phase 4: dQ_inter += dY S0; dK += -diag(exp G) dR S0 + D Delta dS (columns of this half).
        {
          const Split8 AGdR{lds_tr8s(sb + oGdRh + 16 * pw, kLP, lt), lds_tr8s(sb + oGdRl + 16 * pw, kLP, lt)};
          const Split8 ADD{lds_tr8s(sb + oDDh + 16 * pw, kLP, lt), lds_tr8s(sb + oDDl + 16 * pw, kLP, lt)};
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const int c0 = 16 * (4 * hw + t);
            const Split8 B0{lds_tr8s(sb + oS0h + c0, kLS, lt), lds_tr8s(sb + oS0l + c0, kLS, lt)};
            const Split8 B1{lds_tr8s(sb + odSh + c0, kLS, lt), lds_tr8s(sb + odSl + c0, kLS, lt)};
            if constexpr (kExactDy)
              dQi[t] = mma2(dQi[t], dYo.hi, B0);
            else
              dQi[t] = mma3(dQi[t], dYo, B0);
            dK[t] = mma3(dK[t], AGdR, B0);
            dK[t] = mma3(dK[t], ADD, B1);
          }
        }
      };
      int r0 = 0;
      for (; r0 + 32 < a.Dv; r0 += 32) block(r0, std::true_type{});
      block(r0, std::false_type{});

      // End of the state rows for this value head: per-position partials, then the 64 x 64 part.
      int lt = tid;
      asm volatile("" : "+v"(lt));
      const int g = (lt >> 4) & 3, li = lt & 15, pw = (lt >> 6) & 3, hw = lt >> 8, ip = 16 * pw + li;
      const int i0 = 16 * pw + 4 * g;  // first of the lane's accumulator rows
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const float v = sum16(gpart[jj]), h = sum16(hD[jj]), bt = sum16(bpart[jj]);
        // the 16 lanes of a row hold the same bits: no branch
        gpos[hw][i0 + jj] = v, hpos[hw][i0 + jj] = h, bpos[hw][i0 + jj] = bt;
      }
      {
        float v = sum16(sds);
        v = swap32_sum(swap16_sum(v));
        red[tid >> 6] = v;  // every lane of the wave holds the same bits
      }
      __syncthreads();

      // E1: Q rows into the end-phase region. Per lane, at i = ip and j = 16 key_tile(pw, hw, mi) + 4g + jj (dP and
      // dT masked to j <= i): the row and column sums of dP * P (the P factor's part of dG), P * M with
      // M_ij = exp(G_i - G_j) over P's entries into the end-phase region, and dT, both as hi and lo, dT in place of P
      // (each lane rewrites only the P entries it has just read).
      {
        {
#pragma unroll
          for (int q2 = 0; q2 < 2; ++q2) {
            const int e = lt + kThreads * q2;
            *reinterpret_cast<uint4*>(sb + eQb + swz(e >> 4, (e & 15) * 8, kLK)) = __builtin_bit_cast(uint4, nb.ys[q2]);
          }
        }
        // Row sums (over j) add up over g here and over hw in dG; column sums (over i) over li here and over pw in dG.
        float prow = 0.f;
        const float gi = Gf[ip];
#pragma unroll
        for (int mi = 0; mi < 2; ++mi) {
          const int j0 = 16 * key_tile(pw, hw, mi) + 4 * g, at = swz(ip, j0, kLT);
          const uint2 ph = *reinterpret_cast<const uint2*>(PL[0] + at);
          const uint2 pl = *reinterpret_cast<const uint2*>(PL[1] + at);
          const uint32_t hw4[2] = {ph.x, ph.y}, lw4[2] = {pl.x, pl.y};
          float pm[4], db[4];
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const int j = j0 + jj;
            const float dp = j <= ip ? dPt[mi][jj] : 0.f;
            const uint32_t hb = hw4[jj >> 1], lb = lw4[jj >> 1];
            const float pv = jj & 1 ? __uint_as_float(hb & 0xffff0000u) + __uint_as_float(lb & 0xffff0000u)
                                    : __uint_as_float(hb << 16) + __uint_as_float(lb << 16);
            const float x = dp * pv;
            prow += x;
            const float col = sum16(x);
            x2c[pw][j] = col;
            // Where j > i, dp is zero and the exponent positive: clamped at 0 to keep the product finite.
            pm[jj] = dp * __expf(fminf(gi - Gf[j], 0.f));
            db[jj] = j <= ip ? dTt[mi][jj] : 0.f;
          }
          put4(sb + eMh, sb + eMl, at, pm[0], pm[1], pm[2], pm[3]);
          put4(PL[0], PL[1], at, db[0], db[1], db[2], db[3]);
        }
        prow = swap32_sum(swap16_sum(prow));
        x2r[hw][ip] = prow;  // the same bits in the four lane groups
      }
      __syncthreads();

      {  // the next head's tile (ti was staged at this head's start)
        int lq = tid;
        asm volatile("" : "+v"(lq));
        load_tile(ti, nx, nhv, lq);
      }
      // E2: dQ += diag(exp G) dQ_inter and its dG term; K K^T (the first value head only, kept in registers);
      // dQ += (P * M) K; dK += (P * M)^T Q; Z = dT T^T, stored as Z^T.
      {
        float tq[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const int i = i0 + jj, c = 16 * (4 * hw + t) + li;
            tq[jj] += (float)sb[eQb + swz(i, c, kLK)] * dQi[t][jj];
            dQ[t][jj] += gam[i] * dQi[t][jj];
          }
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const float v = sum16(tq[jj]);
          tpos[hw][i0 + jj] = v;
        }
        if (e == cur.e0) {
#pragma unroll
          for (int mi = 0; mi < 2; ++mi) {
            const int m = key_tile(pw, hw, mi);
            kk[mi] = zero4();
            if (m <= pw) {
#pragma unroll
              for (int s = 0; s < 4; ++s)
                kk[mi] = mma(kk[mi], lds8(Kres + swz(ip, 32 * s + 8 * g, kLK)), lds8(Kres + swz(16 * m + li, 32 * s + 8 * g, kLK)));
            }
          }
        }
        // P * M is zero above the diagonal: rows i < 32 end at column 31, and columns j >= 32 start at row 32.
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          if (s == 0 || pw >= 2) {
            const int at = swz(ip, 32 * s + 8 * g, kLT);
            const Split8 Apm{lds8(sb + eMh + at), lds8(sb + eMl + at)};  // (P * M) rows i = ip, k = j
#pragma unroll
            for (int t = 0; t < 4; ++t)
              dQ[t] = mma2(dQ[t], Apm, lds_tr8s(Kres + 32 * s * kLK + 16 * (4 * hw + t), kLK, lt));
          }
          if (s == 1 || pw < 2) {
            const Split8 Apmt{lds_tr8s(sb + eMh + 32 * s * kLT + 16 * pw, kLT, lt),
                              lds_tr8s(sb + eMl + 32 * s * kLT + 16 * pw, kLT, lt)};  // (P * M)^T rows j = ip, k = i
#pragma unroll
            for (int t = 0; t < 4; ++t)
              dK[t] = mma2(dK[t], Apmt, lds_tr8s(sb + eQb + 32 * s * kLK + 16 * (4 * hw + t), kLK, lt));
          }
        }
#pragma unroll
        for (int mi = 0; mi < 2; ++mi) {
          const int mr = 16 * (2 * hw + mi) + li;  // this lane's column m of Z
          f32x4 z = zero4();
#pragma unroll
          for (int s = 0; s < 2; ++s) {
            const int aa = swz(ip, 32 * s + 8 * g, kLT), ab = swz(mr, 32 * s + 8 * g, kLT);
            z = mma3(z, Split8{lds8(PL[0] + aa), lds8(PL[1] + aa)}, Split8{lds8(TL[0] + ab), lds8(TL[1] + ab)});
          }
          put4(sb + eZh, sb + eZl, swz(mr, i0, kLT), z[0], z[1], z[2], z[3]);
        }
      }
      __syncthreads();

      load_rows(nb.xs, a.ckpt, nx, nhv, 0, lt);  // the next head's first S0 rows (nb.xs went to LDS in E1)
      // E3: dA = -T^T Z below the diagonal (rows p = i0 + jj, columns m = 16 key_tile(pw, hw, mi) + li, as kk), and at
      // once its products with E = exp(G_p - G_m) and K K^T: the A part of dbeta (row sums), of dG (row and column
      // sums), and dKK = diag(beta) (dA * E), stored as dKK^T.
      {
        // Only tiles mt <= pw are kept (mcol < p), and T^T rows p >= 32 are zero below column 32.
        Split8 AT[2];  // T^T rows p = ip, k = i
#pragma unroll
        for (int s = 0; s < 2; ++s)
          AT[s] = Split8{lds_tr8s(TL[0] + 32 * s * kLT + 16 * pw, kLT, lt),
                         lds_tr8s(TL[1] + 32 * s * kLT + 16 * pw, kLT, lt)};
        float rowp[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int mi = 0; mi < 2; ++mi) {
          const int mt = key_tile(pw, hw, mi), mcol = 16 * mt + li;
          f32x4 da = zero4();
          if (mt <= pw) {
#pragma unroll
            for (int s = 0; s < 2; ++s) {
              if (s == 1 || pw < 2) {
                const int ab = swz(mcol, 32 * s + 8 * g, kLT);
                da = mma3(da, AT[s], Split8{lds8(sb + eZh + ab), lds8(sb + eZl + ab)});
              }
            }
          }
          float colp = 0.f, kkt[4];
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const int pr = i0 + jj;
            const float e = __expf(fminf(Gf[pr] - Gf[mcol], 0.f));  // finite everywhere; used where mcol < pr
            const float dae = mcol < pr ? -da[jj] * e : 0.f;           // dA_pm E_pm
            const float prod = dae * kk[mi][jj];
            rowp[jj] += prod;
            colp += bet[pr] * prod;
            kkt[jj] = bet[pr] * dae;
          }
          put4(sb + eKh, sb + eKl, swz(mcol, i0, kLT), kkt[0], kkt[1], kkt[2], kkt[3]);
          colp = swap32_sum(swap16_sum(colp));
          x1cp[pw][mcol] = colp;
        }
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const float v = sum16(rowp[jj]);
          dbAp[hw][i0 + jj] = v;
        }
      }
      __syncthreads();

      load_rows(nb.ys, a.dsend, nx, nhv, 0, lt);  // and its first dS rows, dy and v
      load_dy_v(nb, nx, nhv, 0, lt);
      // E4: dK += (dKK + dKK^T) K for rows j = ip, this half's columns: dKK rows j through the transposing read of
      // dKK^T, dKK^T rows j directly.
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int at = swz(ip, 32 * s + 8 * g, kLT);
        const Split8 A1{lds_tr8s(sb + eKh + 32 * s * kLT + 16 * pw, kLT, lt), lds_tr8s(sb + eKl + 32 * s * kLT + 16 * pw, kLT, lt)};
        const Split8 A2{lds8(sb + eKh + at), lds8(sb + eKl + at)};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const bf16x8 B = lds_tr8s(Kres + 32 * s * kLK + 16 * (4 * hw + t), kLK, lt);
          // dKK is strictly lower: dKK[j][i] needs i < j, dKK[i][j] needs i > j.
          if (s == 0 || pw >= 2) dK[t] = mma2(dK[t], A1, B);
          if (s == 1 || pw < 2) dK[t] = mma2(dK[t], A2, B);
        }
      }
      // E5 (one wave): dG per position, dg = its reverse cumulative sum (a suffix scan over the wave), and dbeta.
      if (tid < kC) {
        const int t = tid;
        const float hs = hpos[0][t] + hpos[1][t];
        float hsum = sum16(hs);
        hsum = swap32_sum(swap16_sum(hsum));
        float sds_all = 0.f;
#pragma unroll
        for (int u = 0; u < kThreads / 64; ++u) sds_all += red[u];
        const float dbA = dbAp[0][t] + dbAp[1][t];
        float v = gam[t] * (tpos[0][t] + tpos[1][t]) + gpos[0][t] + gpos[1][t] - hs + bet[t] * dbA -
                  (x1cp[0][t] + x1cp[1][t] + x1cp[2][t] + x1cp[3][t]) + x2r[0][t] + x2r[1][t] -
                  (x2c[0][t] + x2c[1][t] + x2c[2][t] + x2c[3][t]);
        if (t == kC - 1) v += hsum + gam[kC - 1] * sds_all;
#pragma unroll
        for (int off = 1; off < kC; off <<= 1) {
          const float u = __shfl_down(v, off);
          if (t + off < kC) v += u;
        }
        if constexpr (kFused) {
          const int64_t g0 = tok * a.Hv + hv;
          const uint32_t gi = uint32_t(t * a.Hv);
          const float dbT = bpos[0][t] + bpos[1][t];
          float pa = 0.f, pd = 0.f;
          if (t < L) {
            float da, db;
            gate_bwd<bf16_t>(bf16_to_f32(a.pro.a[g0 + gi]), bf16_to_f32(a.pro.b[g0 + gi]), rnd<bf16_t>(dbT + dbA), v,
                             expf(a.pro.a_log[hv]), a.pro.dt_bias[hv], da, db, pa, pd);
            a.pro.da[g0 + gi] = f32_to_bf16(da);
            a.pro.db[g0 + gi] = f32_to_bf16(db);
          }
          pa = sum16(pa), pd = sum16(pd);
          pa = swap32_sum(swap16_sum(pa)), pd = swap32_sum(swap16_sum(pd));
          if (t == 0) a.pro.part[(slot * a.Hv + hv) * 2] = pa, a.pro.part[(slot * a.Hv + hv) * 2 + 1] = pd;
        } else if (t < L) {
          const int64_t g0 = tok * a.Hv + hv;
          const uint32_t gi = uint32_t(t * a.Hv);
          a.dg[g0 + gi] = a.g_is_log ? v : v / a.g[g0 + gi];
          const float dbT = bpos[0][t] + bpos[1][t];
          IO<OutT>::st(static_cast<OutT*>(a.dbeta) + g0, gi, dbT + dbA);
        }
      }
    }

    if constexpr (kSplit) {  // the item's value head's dq and dk, float32, [64][128] each (rows past L unused)
      int lt = tid;
      asm volatile("" : "+v"(lt));
      const int g = (lt >> 4) & 3, li = lt & 15, pw = (lt >> 6) & 3, hw = lt >> 8;
      float* pq = a.dqk_part + (slot * a.Hv + hk * grp + cur.e0) * (2 * kC * Dk);
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int at = (16 * pw + 4 * g + jj) * Dk + 16 * (4 * hw + t) + li;
          pq[at] = dQ[t][jj];
          pq[kC * Dk + at] = dK[t][jj];
        }
      continue;
    }
    if constexpr (kFused) {
      // dq, dk rounded to bf16 into rows [64][128] in the end phase's bytes (E5's reads of them done), then the
      // normalisation's backward row by row, 16 lanes of 8 elements per row as in the separate pass: the raw rows,
      // and the results, through buffer resources that end at the chunk's last row.
      __syncthreads();
      {
        int lt = tid;
        asm volatile("" : "+v"(lt));
        const int g = (lt >> 4) & 3, li = lt & 15, pw = (lt >> 6) & 3, hw = lt >> 8;
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const int at = (16 * pw + 4 * g + jj) * kLK + 16 * (4 * hw + t) + li;
            sb[eQb + at] = static_cast<__bf16>(dQ[t][jj]);
            sb[eQb + kC * kLK + at] = static_cast<__bf16>(dK[t][jj]);
          }
      }
      __syncthreads();
      {
        const uint32_t bytes = uint32_t(L * sk) * 2u;
        const int64_t base = (tok * a.Hk + hk) * Dk;
        const auto qrr = buffer_rsrc(a.pro.q_raw + base, bytes), krr = buffer_rsrc(a.pro.k_raw + base, bytes);
        const auto dqo = buffer_rsrc(static_cast<bf16_t*>(a.dq) + base, bytes);
        const auto dko = buffer_rsrc(static_cast<bf16_t*>(a.dk) + base, bytes);
        const int c8 = (tid & 15) * 8;
        for (int rr = tid >> 4; rr < 2 * kC; rr += kThreads / 16) {
          const bool isk = rr >= kC;
          const int t = rr & (kC - 1);
          const uint32_t off = uint32_t(t * sk + c8) * 2u;
          const uint4 xr = buf_ld16(isk ? krr : qrr, off);
          const uint4 gr = *reinterpret_cast<const uint4*>(sb + eQb + rr * kLK + c8);
          float x[8], gg[8];
          const uint32_t xw[4] = {xr.x, xr.y, xr.z, xr.w}, gw[4] = {gr.x, gr.y, gr.z, gr.w};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            x[2 * j] = __uint_as_float(xw[j] << 16), x[2 * j + 1] = __uint_as_float(xw[j] & 0xffff0000u);
            gg[2 * j] = __uint_as_float(gw[j] << 16), gg[2 * j + 1] = __uint_as_float(gw[j] & 0xffff0000u);
          }
          float ss, gx;
          norm_bwd_sums(x, gg, isk ? a.pro.scale_k : a.pro.scale_q, ss, gx);
          norm_bwd_apply(x, gg, sum16(ss), sum16(gx), Dk);
          buf_st16(isk ? dko : dqo, off,
                   uint4{f32x2_to_bf16x2(x[0], x[1]), f32x2_to_bf16x2(x[2], x[3]), f32x2_to_bf16x2(x[4], x[5]),
                         f32x2_to_bf16x2(x[6], x[7])});
        }
      }
    } else {
    // dq, dk for the wave's positions and columns (lane -> column 16 (4 hw + t) + li, rows 16 pw + 4g + jj), through
    // buffer resources that end at the chunk's last row; lane indices from an opaque copy, so their addresses are
    // formed here rather than hoisted out of the item loop.
      int lt = tid;
      asm volatile("" : "+v"(lt));
      const int g = (lt >> 4) & 3, li = lt & 15, pw = (lt >> 6) & 3, hw = lt >> 8;
      const uint32_t bytes = uint32_t(L * sk) * uint32_t(sizeof(OutT));
      const auto dqr = buffer_rsrc(static_cast<OutT*>(a.dq) + (tok * a.Hk + hk) * Dk, bytes);
      const auto dkr = buffer_rsrc(static_cast<OutT*>(a.dk) + (tok * a.Hk + hk) * Dk, bytes);
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const uint32_t at = uint32_t((16 * pw + 4 * g + jj) * sk + 16 * (4 * hw + t) + li);
          BufIO<OutT>::st(dqr, at, dQ[t][jj]);
          BufIO<OutT>::st(dkr, at, dK[t][jj]);
        }
    }
  }
}

// dA_log and ddt_bias [Hv]: the per-(chunk slot, value head) sums of the fused gradient kernel, summed over the slots.
// One wave per head: lane l sums slots l, l + 64, ... in order, then the wave's lanes are summed in a fixed order, so
// the result does not depend on timing.
__global__ __launch_bounds__(256) void chunk_gate_sums_kernel(const float* part, int64_t NC, int Hv, float* da_log,
                                                              float* ddt_bias) {
  const int h = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (h >= Hv) return;
  float sa = 0.f, sd = 0.f;
  for (int64_t c = lane; c < NC; c += 64) {
    const float2 x = *reinterpret_cast<const float2*>(part + (c * Hv + h) * 2);
    sa += x.x, sd += x.y;
  }
  sa = sum16(sa), sd = sum16(sd);
  sa = swap32_sum(swap16_sum(sa)), sd = swap32_sum(swap16_sum(sd));
  if (lane == 0) da_log[h] = sa, ddt_bias[h] = sd;
}

// dq, dk [tokens, Hk, Dk] of the split gradient kernel: the sum over the key head's value heads, in order, of their
// partials. Thread -> (chunk slot, key head, position, four columns); positions past the chunk's end write nothing.
template <typename OutT>
__global__ __launch_bounds__(256) void chunk_dqk_sum_kernel(ChunkArgs a) {
  constexpr int Dk = 128;
  const int grp = a.Hv / a.Hk;
  const int64_t id = int64_t(blockIdx.x) * 256 + threadIdx.x;
  const int c4 = int(id & 31), t = int((id >> 5) & (kC - 1));
  const int64_t sh = id >> 11;  // slot * Hk + hk
  if (sh >= a.lay.NC * a.Hk) return;
  const int64_t slot = sh / a.Hk;
  const int hk = int(sh % a.Hk);
  const SlotPos sp = slot_pos(a.tab, slot);
  if (t >= sp.L) return;
  float4 q = make_float4(0.f, 0.f, 0.f, 0.f), k = q;
  for (int e = 0; e < grp; ++e) {
    const float* pq = a.dqk_part + (slot * a.Hv + hk * grp + e) * (2 * kC * Dk) + t * Dk + 4 * c4;
    const float4 x = *reinterpret_cast<const float4*>(pq), y = *reinterpret_cast<const float4*>(pq + kC * Dk);
    q.x += x.x, q.y += x.y, q.z += x.z, q.w += x.w;
    k.x += y.x, k.y += y.y, k.z += y.z, k.w += y.w;
  }
  const int64_t at = ((sp.tok + t) * a.Hk + hk) * Dk + 4 * c4;
  OutT* dq = static_cast<OutT*>(a.dq) + at;
  OutT* dk = static_cast<OutT*>(a.dk) + at;
  IO<OutT>::st(dq, 0, q.x), IO<OutT>::st(dq, 1, q.y), IO<OutT>::st(dq, 2, q.z), IO<OutT>::st(dq, 3, q.w);
  IO<OutT>::st(dk, 0, k.x), IO<OutT>::st(dk, 1, k.y), IO<OutT>::st(dk, 2, k.z), IO<OutT>::st(dk, 3, k.w);
}

// The same with the layer's prologue behind (qb_gdn_bwd_prologue): each summed dq and dk row rounded to bf16, as
// the unfused backward stores it, then the q/k normalisation's backward as the separate pass forms it (16 lanes of
// 8 elements per row, the row sums on the 16-lane DPP tree), written as dq_raw and dk_raw. Thread -> (chunk slot,
// key head, position, q or k row, 8 columns).
__global__ __launch_bounds__(256) void chunk_dqk_sum_prologue_kernel(ChunkArgs a) {
  constexpr int Dk = 128;
  const int grp = a.Hv / a.Hk;
  const int64_t id = int64_t(blockIdx.x) * 256 + threadIdx.x, rid = id >> 4;
  const int c8 = int(id & 15) * 8, isk = int(rid & 1), t = int((rid >> 1) & (kC - 1));
  const int64_t sh = rid >> 7;  // slot * Hk + hk; a row's 16 lanes leave together
  if (sh >= a.lay.NC * a.Hk) return;
  const int64_t slot = sh / a.Hk;
  const int hk = int(sh % a.Hk);
  const SlotPos sp = slot_pos(a.tab, slot);
  if (t >= sp.L) return;
  float gg[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int e = 0; e < grp; ++e) {
    const float* pq = a.dqk_part + (slot * a.Hv + hk * grp + e) * (2 * kC * Dk) + isk * kC * Dk + t * Dk + c8;
    const float4 x0 = *reinterpret_cast<const float4*>(pq), x1 = *reinterpret_cast<const float4*>(pq + 4);
    gg[0] += x0.x, gg[1] += x0.y, gg[2] += x0.z, gg[3] += x0.w;
    gg[4] += x1.x, gg[5] += x1.y, gg[6] += x1.z, gg[7] += x1.w;
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) gg[j] = bf16_to_f32(f32_to_bf16(gg[j]));
  const int64_t at = ((sp.tok + t) * a.Hk + hk) * Dk + c8;
  const uint4 xr = *reinterpret_cast<const uint4*>((isk ? a.pro.k_raw : a.pro.q_raw) + at);
  float x[8];
  const uint32_t xw[4] = {xr.x, xr.y, xr.z, xr.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) x[2 * j] = __uint_as_float(xw[j] << 16), x[2 * j + 1] = __uint_as_float(xw[j] & 0xffff0000u);
  float ss, gx;
  norm_bwd_sums(x, gg, isk ? a.pro.scale_k : a.pro.scale_q, ss, gx);
  norm_bwd_apply(x, gg, sum16(ss), sum16(gx), Dk);
  *reinterpret_cast<uint4*>(static_cast<bf16_t*>(isk ? a.dk : a.dq) + at) =
      uint4{f32x2_to_bf16x2(x[0], x[1]), f32x2_to_bf16x2(x[2], x[3]), f32x2_to_bf16x2(x[4], x[5]),
            f32x2_to_bf16x2(x[6], x[7])};
}

}  // namespace

hipError_t launch_chunk_dqk_sum(const ChunkArgs& a, bool out_bf16, hipStream_t s, bool fused_prologue) {
  if (fused_prologue) {
    if (!out_bf16) return hipErrorInvalidValue;
    const int64_t threads = a.lay.NC * a.Hk * kC * 2 * 16;
    if (threads == 0) return hipSuccess;
    hipLaunchKernelGGL(chunk_dqk_sum_prologue_kernel, dim3(unsigned((threads + 255) / 256)), dim3(256), 0, s, a);
    return hipGetLastError();
  }
  const int64_t threads = a.lay.NC * a.Hk * kC * 32;
  if (threads == 0) return hipSuccess;
  const dim3 grid(unsigned((threads + 255) / 256));
  if (out_bf16)
    hipLaunchKernelGGL(chunk_dqk_sum_kernel<bf16_t>, grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(chunk_dqk_sum_kernel<float>, grid, dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t launch_chunk_bwd_grads(const ChunkArgs& a, bool out_bf16, hipStream_t s, bool fused_prologue) {
  const int total = int(a.lay.NC) * a.Hk * (a.dqk_part ? a.Hv / a.Hk : 1);
  if (total == 0) return hipSuccess;
  // One resident block per CU (the kernel's LDS allows no more), looping over its items; a multiple of 8 blocks, so
  // each block's items stay on its XCD.
  int dev = 0, cus = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return e;
  const int grid = total <= cus ? total : (cus >= 8 ? cus & ~7 : cus);
  const bool split = a.dqk_part != nullptr;
  if (fused_prologue) {
    if (!out_bf16) return hipErrorInvalidValue;
    if (split)
      hipLaunchKernelGGL((chunk_bwd_grads_kernel<bf16_t, true, true>), dim3(grid), dim3(kThreads), 0, s, a);
    else
      hipLaunchKernelGGL((chunk_bwd_grads_kernel<bf16_t, true, false>), dim3(grid), dim3(kThreads), 0, s, a);
  } else if (out_bf16) {
    if (split)
      hipLaunchKernelGGL((chunk_bwd_grads_kernel<bf16_t, false, true>), dim3(grid), dim3(kThreads), 0, s, a);
    else
      hipLaunchKernelGGL((chunk_bwd_grads_kernel<bf16_t, false, false>), dim3(grid), dim3(kThreads), 0, s, a);
  } else {
    if (split)
      hipLaunchKernelGGL((chunk_bwd_grads_kernel<float, false, true>), dim3(grid), dim3(kThreads), 0, s, a);
    else
      hipLaunchKernelGGL((chunk_bwd_grads_kernel<float, false, false>), dim3(grid), dim3(kThreads), 0, s, a);
  }
  return hipGetLastError();
}

hipError_t launch_chunk_gate_sums(const ChunkArgs& a, float* da_log, float* ddt_bias, hipStream_t s) {
  hipLaunchKernelGGL(chunk_gate_sums_kernel, dim3((a.Hv + 3) / 4), dim3(256), 0, s, a.pro.part, a.lay.NC, a.Hv,
                     da_log, ddt_bias);
  return hipGetLastError();
}

}  // namespace qbgdn
