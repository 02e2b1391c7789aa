// Chunked design, kernel 4: the per-chunk gradients. One block (4 waves) per (chunk slot, key head); the value heads
// of the key head's GQA group run in order and their dq, dk contributions add up in registers, so the sums over
// value heads have a fixed order (reference src/delta_grad.cpp:194-198) and need no atomics.
//
// Per value head, with S0 the chunk's start state (checkpoint), dS its end-state cotangent (from the backward state
// pass) and the chunk's T, G (from prep), the state rows are streamed in blocks of 32:
//   KS = K S0^T, R = V - diag(exp G) KS, Delta = Tb R, KdS = K dS^T,
//   dDelta = P^T dY + D KdS, dR = Tb^T dDelta                          (Tb = T diag(beta), D = diag(exp(G_63 - G)))
//   dP^T += Delta dY^T, dTb^T += R dDelta^T, dQ_inter += dY S0, dK += -diag(exp G) dR S0 + D Delta dS
// then, once per value head, the 64 x 64 part:
//   dQ += diag(exp G) dQ_inter + (dP * M) K,  dK += (dP * M)^T Q + (dKK + dKK^T) K
//   dA = -T^T (dTb diag(beta)) T^T,  dKK = strict_lower(diag(beta) dA * E)
//   dbeta_j = sum_i dTb_ij T_ij + sum_m dA_jm E_jm (K K^T)_jm,  dG from every exp(.) factor, dg = reverse cumsum
// (tests/chunk_math.py restates these equations and checks them against the oracle.) Wave w owns positions
// 16w..16w+15 of every position-indexed result. MFMA with split float32 operands as in the forward.
#include <type_traits>

#include "chunk_common.h"
#include "chunk_kernels.h"

namespace qbgdn {
namespace {

constexpr int kThreads = 256;
constexpr int kLDK = 128 + kPadB;  // bf16 [.][128] rows
constexpr int kLDC = kC + kPadB;   // bf16 [.][64] rows
constexpr int kLDR = 40;           // bf16 [.][32] rows, padded
constexpr int kLDN = 32;           // bf16 [.][32] rows, packed
constexpr int kLDF = kC + 1;       // f32 [.][64] rows

// Block-loop region (bf16 element offsets).
constexpr int oS0h = 0, oS0l = oS0h + 32 * kLDK;
constexpr int oS0th = oS0l + 32 * kLDK, oS0tl = oS0th + 128 * kLDR;
constexpr int odSh = oS0tl + 128 * kLDR, odSl = odSh + 32 * kLDK;
constexpr int odSth = odSl + 32 * kLDK, odStl = odSth + 128 * kLDR;
constexpr int odYth = odStl + 128 * kLDR, odYtl = odYth + 32 * kLDC;
constexpr int oRth = odYtl + 32 * kLDC, oRtl = oRth + 32 * kLDC;
constexpr int oRmh = oRtl + 32 * kLDC, oRml = oRmh + kC * kLDN;
constexpr int oDmh = oRml + kC * kLDN, oDml = oDmh + kC * kLDN;
constexpr int oDDmh = oDml + kC * kLDN, oDDml = oDDmh + kC * kLDN;
constexpr int odDth = oDDml + kC * kLDN, odDtl = odDth + 32 * kLDC;
constexpr int odDmh = odDtl + 32 * kLDC, odDml = odDmh + kC * kLDN;
constexpr int oGdRh = odDml + kC * kLDN, oGdRl = oGdRh + kC * kLDN;
constexpr int kLoopBytes = (oGdRl + kC * kLDN) * 2;
// End-phase region (aliases the block-loop region): bf16 K, Q then f32 64 x 64 matrices.
constexpr int eKb = 0, eQb = kC * kLDK;                    // bf16 offsets
constexpr int eF = (2 * kC * kLDK * 2) / 4;                // first f32 offset
constexpr int edPM = eF, eQK = edPM + kC * kLDF, edTb = eQK + kC * kLDF, eT = edTb + kC * kLDF;
constexpr int eKK = eT + kC * kLDF, eZt = eKK + kC * kLDF;
constexpr int kEndBytes = (eZt + kC * kLDF) * 4;
constexpr int kSmemBytes = kLoopBytes > kEndBytes ? kLoopBytes : kEndBytes;

__device__ __forceinline__ void put_split(__bf16* hi, __bf16* lo, int at, float x) {
  const __bf16 h = (__bf16)x;
  hi[at] = h;
  lo[at] = (__bf16)(x - (float)h);
}

template <typename OutT>
__global__ __launch_bounds__(kThreads) void chunk_bwd_grads_kernel(ChunkArgs a) {
  constexpr int Dk = 128;
  constexpr bool kExactDy = std::is_same<OutT, bf16_t>::value;
  __shared__ __align__(16) unsigned char smem[kSmemBytes];
  __shared__ double Gd[kC];
  __shared__ float gam[kC], Dd[kC], Bs[kC], dGpos[kC], hDtot[kC], x1r[kC], x1c[kC], x2r[kC], x2c[kC];
  __shared__ float dbT[kC], dbA[kC], dGt[kC], red[kThreads];
  __shared__ float SdS_total;
  __bf16* sb = reinterpret_cast<__bf16*>(smem);
  float* sf = reinterpret_cast<float*>(smem);

  const int total = int(a.lay.NC) * a.Hk;
  const int wid = xcd_remap(blockIdx.x, total);
  const int64_t slot = wid / a.Hk;
  const int hk = wid % a.Hk, grp = a.Hv / a.Hk;
  const SlotPos sp = slot_pos(a.tab, slot);
  const int L = sp.L;
  const int64_t tok = sp.tok;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, li = lane & 15;
  const OutT* dy = static_cast<const OutT*>(a.dy);

  // K and Q rows of the wave's positions (A operands), and Q K^T with lane -> column j = 16w + li, rows i.
  stage_rows_bf16<Dk>(sb + eKb, kLDK, a.k, tok, a.Hk, hk, L, kThreads);
  stage_rows_bf16<Dk>(sb + eQb, kLDK, a.q, tok, a.Hk, hk, L, kThreads);
  __syncthreads();
  bf16x8 Kf[4], Qf[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    Kf[s] = lds8(sb + eKb + (16 * w + li) * kLDK + 32 * s + 8 * g);
    Qf[s] = lds8(sb + eQb + (16 * w + li) * kLDK + 32 * s + 8 * g);
  }
  f32x4 qk[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    qk[m] = zero4();
    if (m >= w) {
#pragma unroll
      for (int s = 0; s < 4; ++s) qk[m] = mma(qk[m], lds8(sb + eQb + (16 * m + li) * kLDK + 32 * s + 8 * g), Kf[s]);
    }
  }
  f32x4 dQ[8], dK[8];
#pragma unroll
  for (int t = 0; t < 8; ++t) dQ[t] = zero4(), dK[t] = zero4();

  for (int e = 0; e < grp; ++e) {
    const int hv = hk * grp + e;
    const int64_t sh = slot * a.Hv + hv;
    __syncthreads();
    if (tid < kC) {
      const double* G = a.Gall + sh * kC;
      const double gt = G[tid], gl = G[kC - 1];
      Gd[tid] = gt;
      gam[tid] = expf(float(gt));
      Dd[tid] = expf(float(gl - gt));
      Bs[tid] = tid < L ? bf16_to_f32(a.beta[(tok + tid) * a.Hv + hv]) : 0.f;
    }
    __syncthreads();
    const float* T = a.Tall + sh * int64_t(kC * kC);
    Split8 TbA[2], TbtA[2], PA[2];
    {
      const int i = 16 * w + li;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        float x[8], y[8], p[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int jj = 32 * s + 8 * g + j;
          x[j] = T[i * kC + jj] * Bs[jj];
          y[j] = T[jj * kC + i] * Bs[i];
        }
        // P^T row j = i (k = query positions in the stacked order of qk[2s], qk[2s + 1])
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int q0 = 32 * s + 4 * g + jj, q1 = q0 + 16;
          p[jj] = q0 >= i ? qk[2 * s][jj] * expf(float(Gd[q0] - Gd[i])) : 0.f;
          p[4 + jj] = q1 >= i ? qk[2 * s + 1][jj] * expf(float(Gd[q1] - Gd[i])) : 0.f;
        }
        TbA[s] = split8(x);
        TbtA[s] = split8(y);
        PA[s] = split8(p);
      }
    }
    f32x4 dPt[4], dTbt[4], dQi[8];
#pragma unroll
    for (int t = 0; t < 4; ++t) dPt[t] = zero4(), dTbt[t] = zero4();
#pragma unroll
    for (int t = 0; t < 8; ++t) dQi[t] = zero4();
    float gpart[4] = {0.f, 0.f, 0.f, 0.f}, hD[4] = {0.f, 0.f, 0.f, 0.f}, sds = 0.f;

    for (int r0 = 0; r0 < a.Dv; r0 += 32) {
      __syncthreads();
      {  // S0 and dS rows r0..r0+31: thread -> row tid / 8, columns 16 (tid % 8) ..
        const int r = tid >> 3, c0 = (tid & 7) * 16;
        const int64_t at = (sh * a.Dv + r0 + r) * Dk + c0;
        const float* s0p = a.ckpt + at;
        const float* dsp = a.dsend + at;
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const float4 x4 = *reinterpret_cast<const float4*>(s0p + 4 * q4);
          const float4 y4 = *reinterpret_cast<const float4*>(dsp + 4 * q4);
          const float xs[4] = {x4.x, x4.y, x4.z, x4.w}, ys[4] = {y4.x, y4.y, y4.z, y4.w};
#pragma unroll
          for (int u = 0; u < 4; ++u) {
            const int c = c0 + 4 * q4 + u;
            sds += xs[u] * ys[u];
            put_split(sb + oS0h, sb + oS0l, r * kLDK + c, xs[u]);
            put_split(sb + oS0th, sb + oS0tl, c * kLDR + r, xs[u]);
            put_split(sb + odSh, sb + odSl, r * kLDK + c, ys[u]);
            put_split(sb + odSth, sb + odStl, c * kLDR + r, ys[u]);
          }
        }
      }
      {  // dY^T [r][i]: thread -> position tid / 4, rows 8 (tid % 4) ..
        const int i = tid >> 2, r8 = (tid & 3) * 8;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const float x = i < L ? IO<OutT>::ld(dy, ((tok + i) * a.Hv + hv) * a.Dv + r0 + r8 + j) : 0.f;
          put_split(sb + odYth, sb + odYtl, (r8 + j) * kLDC + i, x);
        }
      }
      // The wave's own dY rows (i = 16w + li, k = r = 8g..): A of dY S0, B of Delta dY^T.
      Split8 dYo;
      {
        const int i = 16 * w + li;
        float x[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) x[j] = i < L ? IO<OutT>::ld(dy, ((tok + i) * a.Hv + hv) * a.Dv + r0 + 8 * g + j) : 0.f;
        dYo = split8(x);
      }
      __syncthreads();

      // Phase 1: KS, QS, KdS for positions 16w.. (lane -> column r = 16nt + li, rows i = 16w + 4g + jj).
      f32x4 ks[2], qs[2], kds[2];
      float gks[2][4];
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        ks[nt] = qs[nt] = kds[nt] = zero4();
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const int at = (16 * nt + li) * kLDK + 32 * s + 8 * g;
          const bf16x8 bh = lds8(sb + oS0h + at), bl = lds8(sb + oS0l + at);
          ks[nt] = mma(mma(ks[nt], Kf[s], bh), Kf[s], bl);
          qs[nt] = mma(mma(qs[nt], Qf[s], bh), Qf[s], bl);
          kds[nt] = mma(mma(kds[nt], Kf[s], lds8(sb + odSh + at)), Kf[s], lds8(sb + odSl + at));
        }
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int i = 16 * w + 4 * g + jj, r = 16 * nt + li;
          const float vv = i < L ? bf16_to_f32(a.v[((tok + i) * a.Hv + hv) * a.Dv + r0 + r]) : 0.f;
          gks[nt][jj] = gam[i] * ks[nt][jj];
          const float R = vv - gks[nt][jj];
          const float dyv = (float)sb[odYth + r * kLDC + i] + (float)sb[odYtl + r * kLDC + i];
          gpart[jj] += gam[i] * dyv * qs[nt][jj];
          put_split(sb + oRth, sb + oRtl, r * kLDC + i, R);
          put_split(sb + oRmh, sb + oRml, i * kLDN + r, R);
        }
      }
      __syncthreads();

      // Phase 2: Delta = Tb R and dDelta = P^T dY + D KdS for positions 16w..
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        const int r = 16 * nt + li;
        f32x4 dl = zero4(), dd;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const int at = r * kLDC + 32 * s + 8 * g;
          dl = mma3(dl, TbA[s], Split8{lds8(sb + oRth + at), lds8(sb + oRtl + at)});
        }
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) dd[jj] = Dd[16 * w + 4 * g + jj] * kds[nt][jj];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          if (2 * s + 1 >= w) {
            const int at = r * kLDC + 32 * s + 4 * g;
            if constexpr (kExactDy)
              dd = mma2(dd, PA[s], lds4x2(sb + odYth + at));
            else
              dd = mma3(dd, PA[s], Split8{lds4x2(sb + odYth + at), lds4x2(sb + odYtl + at)});
          }
        }
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int i = 16 * w + 4 * g + jj;
          hD[jj] += Dd[i] * dl[jj] * kds[nt][jj];
          put_split(sb + oDmh, sb + oDml, i * kLDN + r, dl[jj]);
          put_split(sb + oDDmh, sb + oDDml, i * kLDN + r, Dd[i] * dl[jj]);
          put_split(sb + odDth, sb + odDtl, r * kLDC + i, dd[jj]);
          put_split(sb + odDmh, sb + odDml, i * kLDN + r, dd[jj]);
        }
      }
      __syncthreads();

      // Phase 3: dR = Tb^T dDelta; dP^T += Delta dY^T and dTb^T += R dDelta^T (rows j, columns i = own).
#pragma unroll
      for (int nt = 0; nt < 2; ++nt) {
        const int r = 16 * nt + li;
        f32x4 dr = zero4();
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          const int at = r * kLDC + 32 * s + 8 * g;
          dr = mma3(dr, TbtA[s], Split8{lds8(sb + odDth + at), lds8(sb + odDtl + at)});
        }
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int i = 16 * w + 4 * g + jj;
          gpart[jj] -= dr[jj] * gks[nt][jj];
          put_split(sb + oGdRh, sb + oGdRl, i * kLDN + r, -gam[i] * dr[jj]);
        }
      }
      {
        const int atn = (16 * w + li) * kLDN + 8 * g;
        const Split8 BdD{lds8(sb + odDmh + atn), lds8(sb + odDml + atn)};
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          if (m <= w) {
            const int at = (16 * m + li) * kLDN + 8 * g;
            const Split8 AD{lds8(sb + oDmh + at), lds8(sb + oDml + at)};
            if constexpr (kExactDy)
              dPt[m] = mma2(dPt[m], AD, dYo.hi);
            else
              dPt[m] = mma3(dPt[m], AD, dYo);
            dTbt[m] = mma3(dTbt[m], Split8{lds8(sb + oRmh + at), lds8(sb + oRml + at)}, BdD);
          }
        }
      }
      __syncthreads();

      // Phase 4: dQ_inter += dY S0; dK += -diag(exp G) dR S0 + D Delta dS (rows i = own, columns c).
      {
        const int at = (16 * w + li) * kLDN + 8 * g;
        const Split8 AGdR{lds8(sb + oGdRh + at), lds8(sb + oGdRl + at)};
        const Split8 ADD{lds8(sb + oDDmh + at), lds8(sb + oDDml + at)};
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          const int bt = (16 * t + li) * kLDR + 8 * g;
          const Split8 B0{lds8(sb + oS0th + bt), lds8(sb + oS0tl + bt)};
          const Split8 B1{lds8(sb + odSth + bt), lds8(sb + odStl + bt)};
          if constexpr (kExactDy)
            dQi[t] = mma2(dQi[t], dYo.hi, B0);
          else
            dQi[t] = mma3(dQi[t], dYo, B0);
          dK[t] = mma3(dK[t], AGdR, B0);
          dK[t] = mma3(dK[t], ADD, B1);
        }
      }
    }
    // End of the state rows for this value head.
#pragma unroll
    for (int t = 0; t < 8; ++t)
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) dQ[t][jj] += gam[16 * w + 4 * g + jj] * dQi[t][jj];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const float v = sum16(gpart[jj]), h = sum16(hD[jj]);
      if (li == 0) {
        dGpos[16 * w + 4 * g + jj] = v - h;
        hDtot[16 * w + 4 * g + jj] = h;
      }
    }
    red[tid] = sds;
    __syncthreads();

    // E1: K, Q, T, dP * M, dTb, Q K^T into the end-phase region.
    stage_rows_bf16<Dk>(sb + eKb, kLDK, a.k, tok, a.Hk, hk, L, kThreads);
    stage_rows_bf16<Dk>(sb + eQb, kLDK, a.q, tok, a.Hk, hk, L, kThreads);
    for (int q = tid; q < kC * kC; q += kThreads) sf[eT + (q >> 6) * kLDF + (q & 63)] = T[q];
    {
      const int i = 16 * w + li;
#pragma unroll
      for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int j = 16 * m + 4 * g + jj;
          sf[edPM + i * kLDF + j] = j <= i ? dPt[m][jj] * expf(float(Gd[i] - Gd[j])) : 0.f;
          sf[edTb + i * kLDF + j] = j <= i ? dTbt[m][jj] : 0.f;
          // qk: lane -> column j' = 16w + li, rows i' = 16m + 4g + jj
          const int jq = 16 * w + li, iq = 16 * m + 4 * g + jj;
          sf[eQK + iq * kLDF + jq] = iq >= jq ? qk[m][jj] : 0.f;
        }
    }
    __syncthreads();

    // E2: K K^T rows p = own; dQ += (dP * M) K; dK += (dP * M)^T Q; Z = (dTb diag(beta)) T^T.
    {
      const int p = 16 * w + li;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        f32x4 kk = zero4();
        if (mt <= w) {
#pragma unroll
          for (int s = 0; s < 4; ++s) kk = mma(kk, Kf[s], lds8(sb + eKb + (16 * mt + li) * kLDK + 32 * s + 8 * g));
        }
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) sf[eKK + (16 * w + 4 * g + jj) * kLDF + 16 * mt + li] = kk[jj];
      }
      Split8 AdPM[2], AdPMt[2], AdT[2];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        float x[8], y[8], z[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int jj = 32 * s + 8 * g + j;
          x[j] = sf[edPM + p * kLDF + jj];
          y[j] = sf[edPM + jj * kLDF + p];
          z[j] = sf[edTb + p * kLDF + jj] * Bs[jj];
        }
        AdPM[s] = split8(x);
        AdPMt[s] = split8(y);
        AdT[s] = split8(z);
      }
#pragma unroll
      for (int t = 0; t < 8; ++t) {
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          bf16x8 bk, bq;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            bk[j] = sb[eKb + (32 * s + 8 * g + j) * kLDK + 16 * t + li];
            bq[j] = sb[eQb + (32 * s + 8 * g + j) * kLDK + 16 * t + li];
          }
          dQ[t] = mma2(dQ[t], AdPM[s], bk);
          dK[t] = mma2(dK[t], AdPMt[s], bq);
        }
      }
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        f32x4 z = zero4();
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          float tv[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) tv[j] = sf[eT + (16 * mt + li) * kLDF + 32 * s + 8 * g + j];
          z = mma3(z, AdT[s], split8(tv));
        }
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) sf[eZt + (16 * mt + li) * kLDF + 16 * w + 4 * g + jj] = z[jj];
      }
    }
    if (tid < kC) {
      const int j = tid;
      float acc = 0.f;
      for (int i = j; i < kC; ++i) acc += sf[edTb + i * kLDF + j] * sf[eT + i * kLDF + j];
      dbT[j] = acc;
    } else if (tid < 2 * kC) {
      const int i = tid - kC;
      float acc = 0.f;
      for (int j = 0; j <= i; ++j) acc += sf[edPM + i * kLDF + j] * sf[eQK + i * kLDF + j];
      x2r[i] = acc;
    } else if (tid < 3 * kC) {
      const int j = tid - 2 * kC;
      float acc = 0.f;
      for (int i = j; i < kC; ++i) acc += sf[edPM + i * kLDF + j] * sf[eQK + i * kLDF + j];
      x2c[j] = acc;
    } else if (tid == 3 * kC) {
      float acc = 0.f;
      for (int t = 0; t < kThreads; ++t) acc += red[t];
      SdS_total = acc;
    }
    __syncthreads();

    // E3: dA = -T^T Z (strict lower), rows p = own, into the dP * M slot.
    {
      const int p = 16 * w + li;
      Split8 AT[2];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        float x[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) x[j] = sf[eT + (32 * s + 8 * g + j) * kLDF + p];
        AT[s] = split8(x);
      }
      f32x4 da[4];
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) {
        da[mt] = zero4();
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          float zv[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) zv[j] = sf[eZt + (16 * mt + li) * kLDF + 32 * s + 8 * g + j];
          da[mt] = mma3(da[mt], AT[s], split8(zv));
        }
      }
      __syncthreads();  // every wave has read dP * M (E2) and Z before dA overwrites the slot
#pragma unroll
      for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int pr = 16 * w + 4 * g + jj, m = 16 * mt + li;
          sf[edPM + pr * kLDF + m] = m < pr ? -da[mt][jj] : 0.f;
        }
    }
    __syncthreads();

    // E4: dbeta (A part), the A-factor terms of dG, and dKK = beta_p dA E into the dTb slot.
    if (tid < kC) {
      const int p = tid;
      float acc = 0.f;
      for (int m = 0; m < p; ++m)
        acc += sf[edPM + p * kLDF + m] * expf(float(Gd[p] - Gd[m])) * sf[eKK + p * kLDF + m];
      dbA[p] = acc;
      x1r[p] = Bs[p] * acc;
    } else if (tid < 2 * kC) {
      const int m = tid - kC;
      float acc = 0.f;
      for (int p = m + 1; p < kC; ++p)
        acc += Bs[p] * sf[edPM + p * kLDF + m] * expf(float(Gd[p] - Gd[m])) * sf[eKK + p * kLDF + m];
      x1c[m] = acc;
    }
    for (int q = tid; q < kC * kC; q += kThreads) {
      const int p = q >> 6, m = q & 63;
      sf[edTb + p * kLDF + m] = m < p ? Bs[p] * sf[edPM + p * kLDF + m] * expf(float(Gd[p] - Gd[m])) : 0.f;
    }
    __syncthreads();

    // E5: dK += (dKK + dKK^T) K for rows j = own.
    {
      const int j0 = 16 * w + li;
      Split8 A[2];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        float x[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int m = 32 * s + 8 * g + j;
          x[j] = sf[edTb + j0 * kLDF + m] + sf[edTb + m * kLDF + j0];
        }
        A[s] = split8(x);
      }
#pragma unroll
      for (int t = 0; t < 8; ++t)
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          bf16x8 bk;
#pragma unroll
          for (int j = 0; j < 8; ++j) bk[j] = sb[eKb + (32 * s + 8 * g + j) * kLDK + 16 * t + li];
          dK[t] = mma2(dK[t], A[s], bk);
        }
    }
    // E6: dG per position, then dg = reverse cumsum and dbeta.
    if (tid < kC) {
      const int t = tid;
      float v = dGpos[t] + x1r[t] - x1c[t] + x2r[t] - x2c[t];
      if (t == kC - 1) {
        float hsum = 0.f;
        for (int i = 0; i < kC; ++i) hsum += hDtot[i];
        v += hsum + gam[kC - 1] * SdS_total;
      }
      dGt[t] = v;
    }
    __syncthreads();
    if (tid < L) {
      const int t = tid;
      float da = 0.f;
      for (int i = kC - 1; i >= t; --i) da += dGt[i];
      const int64_t gi = (tok + t) * a.Hv + hv;
      a.dg[gi] = a.g_is_log ? da : da / a.g[gi];
      IO<OutT>::st(static_cast<OutT*>(a.dbeta), gi, dbT[t] + dbA[t]);
    }
  }

  // dq, dk for the wave's positions (lane -> column c = 16t + li, rows i = 16w + 4g + jj).
  OutT* dq = static_cast<OutT*>(a.dq);
  OutT* dk = static_cast<OutT*>(a.dk);
#pragma unroll
  for (int t = 0; t < 8; ++t)
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int i = 16 * w + 4 * g + jj;
      if (i < L) {
        const int64_t at = ((tok + i) * a.Hk + hk) * Dk + 16 * t + li;
        IO<OutT>::st(dq, at, dQ[t][jj]);
        IO<OutT>::st(dk, at, dK[t][jj]);
      }
    }
}

}  // namespace

hipError_t launch_chunk_bwd_grads(const ChunkArgs& a, bool out_bf16, hipStream_t s) {
  const int total = int(a.lay.NC) * a.Hk;
  if (total == 0) return hipSuccess;
  if (out_bf16)
    hipLaunchKernelGGL(chunk_bwd_grads_kernel<bf16_t>, dim3(total), dim3(kThreads), 0, s, a);
  else
    hipLaunchKernelGGL(chunk_bwd_grads_kernel<float>, dim3(total), dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace qbgdn
