// Chunked design, kernel 1 (prep), one block per (chunk slot, value head), or per (chunk slot, key head) when that
// grid would not fit on the device at once: everything about the chunk that does not depend on the state, written
// once as MFMA-ready operands (the Tile record, chunk_common.h: T and P as bf16 hi/lo pairs of their
// lower-triangular blocks).
//   G = cumsum of the log-decays (fp64, so G_i - G_j keeps its bits when |G| is large)
//   A = strict_lower(diag(beta) (E * K K^T)),  T = (I + A)^-1
//   P = lower_incl(E * Q K^T),  E_ij = exp(G_i - G_j)
// T is the UT transform of the chunk's delta rule: Delta = T diag(beta) (V - diag(exp G) K S0^T) gives every step's
// delta_t = beta_t (v_t - u_t) of the recurrence (reference src/delta_grad.cpp:14) at once. K K^T and Q K^T run on
// MFMA (bf16 inputs are exact, fp32 accumulation); the inverse is blocked forward substitution in fp32: each 16 x 16
// diagonal block by substitution with the column held in registers, then T_IJ = -T_II sum_K A_IK T_KJ by distance.
#include "chunk_common.h"
#include "chunk_kernels.h"
#include "prologue_math.h"

namespace qbgdn {
namespace {

constexpr int kThreads = 256;
constexpr double kLogFloor = -150.0;
constexpr int kLDK = 144;  // bf16 row stride for Dk = 128: 16-byte aligned rows on staggered banks

typedef short s16x4 __attribute__((ext_vector_type(4)));

// v_mfma_f32_16x16x16_bf16: lane l holds A[l % 16][4 (l / 16) + j], B[4 (l / 16) + j][l % 16], j = 0..3.
__device__ __forceinline__ f32x4 mma16(f32x4 c, s16x4 a, s16x4 b) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}

// LDS: k and q rows while K K^T and Q K^T run; then, in the same bytes, A and T in float32 and P as bf16 hi/lo,
// each as its ten lower-triangular blocks. About 37 KB, so four blocks share a CU. P is laid out as in the tile
// (tri_off), to be copied out as it is; A and T, which stay in LDS, are padded (tri_pad): rows of 20 floats inside a
// block, so that a row's 4 columns written from each of 16 lanes, and the 16 rows of a column read at once, fall on
// distinct banks, and blocks 324 floats apart, so that the four diagonal blocks the substitution reads side by side
// do too.
constexpr int kLdPad = 20, kBlkPad = 16 * kLdPad + 4, kTriPad = 10 * kBlkPad;
__device__ __forceinline__ int tri_pad(int i, int j) {
  return ((i >> 4) * ((i >> 4) + 1) / 2 + (j >> 4)) * kBlkPad + (i & 15) * kLdPad + (j & 15);
}
constexpr int kKQBytes = 2 * kC * kLDK * 2;
constexpr int kAoff = 0, kToff = kTriPad * 4, kPoff = 2 * kTriPad * 4;  // byte offsets of A, T, P (hi then lo)
static_assert(kPoff + 2 * kTri * 2 <= kKQBytes, "A, T and P fit in the k/q staging bytes");

// kFused: the layer's prologue in front (qb_gdn_fwd_prologue). The block reads q_raw, k_raw, a and b in place of
// q, k, g and beta and forms them as the separate prologue pass does, bit for bit (prologue_math.h; a row's sum of
// squares is the same in-lane sum over 8 consecutive elements and DPP reduction over its 16 lanes). It writes beta and
// the log-decay of each of its value heads, and the block of a key head's first value head writes q and k.
//
// hpb: value heads per block, 1 or the key head's whole group (Hv / Hk). A block forms K K^T and Q K^T once for its
// heads and then works through them in turn.
template <bool kFused>
__global__ __launch_bounds__(kThreads) void chunk_prep_kernel(ChunkArgs a, int hpb) {
  __shared__ __align__(16) unsigned char smem[kKQBytes];
  __shared__ double Gd[kC];
  __shared__ float Bs[kC];
  __bf16* Kb = reinterpret_cast<__bf16*>(smem);  // [kC][kLDK]
  __bf16* Qb = Kb + kC * kLDK;
  float* Am = reinterpret_cast<float*>(smem + kAoff);
  float* Tm = reinterpret_cast<float*>(smem + kToff);
  __bf16* Pp = reinterpret_cast<__bf16*>(smem + kPoff);  // hi; lo at + kTri

  const int units = a.Hv / hpb, total = int(a.lay.NC) * units, grp = a.Hv / a.Hk;
  const int wid = xcd_remap(blockIdx.x, total);
  const int64_t slot = wid / units;
  const int hv0 = (wid % units) * hpb, hk = hv0 / grp;
  const SlotPos sp = slot_pos(a.tab, slot);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, li = lane & 15;

  // A value head's log-decay and beta for the chunk's rows (one wave), through buffer resources that end at the
  // chunk's last row (rows past it read as zeros).
  const uint32_t L = uint32_t(sp.L);
  auto load_scalars = [&](const int hv, float& gx, float& bx) {
    const int64_t s0 = sp.tok * a.Hv + hv;
    const uint32_t n = L == 0 ? 0u : (L - 1) * uint32_t(a.Hv) + 1;  // elements from s0 to the chunk's last row
    if constexpr (kFused) {
      const auto ar = buffer_rsrc(a.pro.a + s0, n * 2u), br = buffer_rsrc(a.pro.b + s0, n * 2u);
      const float av = bf16_to_f32(buf_ld2(ar, uint32_t(tid * a.Hv) * 2));
      const float bv = bf16_to_f32(buf_ld2(br, uint32_t(tid * a.Hv) * 2));
      gx = gate_log_decay<bf16_t>(av, a.pro.a_log[hv], a.pro.dt_bias[hv]);
      bx = gate_beta<bf16_t>(bv);
      if (uint32_t(tid) < L) {
        a.pro.log_decay[s0 + int64_t(tid) * a.Hv] = gx;
        a.pro.beta[s0 + int64_t(tid) * a.Hv] = f32_to_bf16(bx);
      }
    } else {
      const auto gr = buffer_rsrc(a.g + s0, n * 4u);
      const auto br = buffer_rsrc(a.beta + s0, n * 2u);
      gx = buf_ld4(gr, uint32_t(tid * a.Hv) * 4);
      bx = bf16_to_f32(buf_ld2(br, uint32_t(tid * a.Hv) * 2));
    }
  };
  float gx = 0.f, bx = 0.f;
  if (tid < kC) load_scalars(hv0, gx, bx);
  // The key head's K and Q rows, read once for every value head of its group; all issued before any is used.
  {
    const int sk = a.Hk * 128;
    const uint32_t bytes = L * uint32_t(sk) * 2u;
    const bf16_t* kb = kFused ? a.pro.k_raw : a.k;
    const bf16_t* qb = kFused ? a.pro.q_raw : a.q;
    const auto kr = buffer_rsrc(kb + sp.tok * sk + hk * 128, bytes);
    const auto qr = buffer_rsrc(qb + sp.tok * sk + hk * 128, bytes);
    uint4 kv[4], qv[4];
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int e = tid + kThreads * q4, t = e >> 4, c8 = (e & 15) * 8;
      kv[q4] = buf_ld16(kr, uint32_t(t * sk + c8) * 2);
      qv[q4] = buf_ld16(qr, uint32_t(t * sk + c8) * 2);
    }
    if constexpr (kFused) {
      // Normalise each row (16 lanes of 8 elements); rows past the chunk's end are zeros and stay zeros. The block
      // of the group's first value head writes them.
      const bool writer = hv0 % grp == 0;
      const auto ko = buffer_rsrc(a.pro.k + sp.tok * sk + hk * 128, bytes);
      const auto qo = buffer_rsrc(a.pro.q + sp.tok * sk + hk * 128, bytes);
      auto norm = [&](uint4& u, float s) {
        float x[8];
        const uint32_t w4[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
        for (int j = 0; j < 4; ++j)
          x[2 * j] = __uint_as_float(w4[j] << 16), x[2 * j + 1] = __uint_as_float(w4[j] & 0xffff0000u);
        norm_row8<bf16_t>(x, sum16(sumsq8(x)), 128, s);
        u = uint4{f32x2_to_bf16x2(x[0], x[1]), f32x2_to_bf16x2(x[2], x[3]), f32x2_to_bf16x2(x[4], x[5]),
                  f32x2_to_bf16x2(x[6], x[7])};
      };
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const int e = tid + kThreads * q4, t = e >> 4, c8 = (e & 15) * 8;
        norm(kv[q4], a.pro.scale_k);
        norm(qv[q4], a.pro.scale_q);
        if (writer) {
          buf_st16(ko, uint32_t(t * sk + c8) * 2, kv[q4]);
          buf_st16(qo, uint32_t(t * sk + c8) * 2, qv[q4]);
        }
      }
    }
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int e = tid + kThreads * q4, t = e >> 4, c8 = (e & 15) * 8;
      *reinterpret_cast<uint4*>(Kb + t * kLDK + c8) = kv[q4];
      *reinterpret_cast<uint4*>(Qb + t * kLDK + c8) = qv[q4];
    }
  }
  __syncthreads();

  // The ten lower-triangular 16 x 16 blocks (I, J) of K K^T and Q K^T, block b = tri_off order, round-robin over the
  // waves (three, three, two, two), on MFMA, formed transposed (K_J K_I^T, K_J Q_I^T) so that a lane holds row
  // i = 16 I + li, columns j = 16 J + 4g + jj: its four values of a row leave as one vector store. They stay in
  // registers for every value head of the group; A and P take the k and q rows' bytes once every wave is done.
  f32x4 kk[3], qk[3];
#pragma unroll
  for (int u = 0; u < 3; ++u) {
    const int b = w + 4 * u;
    const int I = (b >= 1) + (b >= 3) + (b >= 6), J = b - I * (I + 1) / 2;
    kk[u] = zero4(), qk[u] = zero4();
    if (b < 10) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const bf16x8 ak = lds8(Kb + (16 * J + li) * kLDK + 32 * s + 8 * g);
        kk[u] = mma(kk[u], ak, lds8(Kb + (16 * I + li) * kLDK + 32 * s + 8 * g));
        qk[u] = mma(qk[u], ak, lds8(Qb + (16 * I + li) * kLDK + 32 * s + 8 * g));
      }
    }
  }

  for (int vh = 0; vh < hpb; ++vh) {
    const int hv = hv0 + vh;
    Tile* tile = a.tiles + (slot * a.Hv + hv);
    // The thread's indices re-formed from an opaque copy of its id, so that the compiler does not keep the LDS
    // addresses of one head's inverse in registers for the next (they would take the registers of two more waves).
    int tidv = threadIdx.x;
    asm volatile("" : "+v"(tidv));
    const int tid = tidv, lane = tid & 63, w = tid >> 6, g = lane >> 4, li = lane & 15;
    // The first pass: every wave is done with the k and q rows. Later ones: done with the previous head's G, beta,
    // A, T and P.
    __syncthreads();
    // One wave: G = the inclusive prefix sum of the log-decays, accumulated in fp64 by a shuffle scan (so G_i - G_j
    // keeps its bits when |G| is large). Then the next value head's scalars are read, to arrive during this head.
    if (tid < kC) {
      const int t = tid;
      // The log-decay floored at -150: a factor of 0 (or a log-decay of -inf) would make G_i - G_j NaN on every pair
      // across it; at -150 each exp(.) across it is 0 in float32, as the factor 0 makes it.
      double G = uint32_t(t) < L ? fmax(kFused || a.g_is_log ? double(gx) : double(logf(gx)), kLogFloor) : 0.0;
#pragma unroll
      for (int off = 1; off < kC; off <<= 1) {
        const double u = __shfl_up(G, off);
        if (t >= off) G += u;
      }
      const double Glast = __shfl(G, kC - 1);
      Gd[t] = G;
      Bs[t] = uint32_t(t) < L ? bx : 0.f;
      tile->beta[t] = Bs[t];
      tile->gam[t] = expf(float(G));
      tile->dec[t] = expf(float(Glast - G));
      tile->G[t] = float(G);
      if (vh + 1 < hpb) load_scalars(hv + 1, gx, bx);
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < 3; ++u) {
      const int b = w + 4 * u;
      if (b < 10) {
        const int I = (b >= 1) + (b >= 3) + (b >= 6), J = b - I * (I + 1) / 2;
        const int i = 16 * I + li, j0 = 16 * J + 4 * g;
        float av[4], pv[4];
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int j = j0 + jj;
          // The hardware exponential: its error (a few ulp) is far below the 2^-17 of the hi/lo split that carries E.
          const float e = j <= i ? __expf(float(Gd[i] - Gd[j])) : 0.f;
          av[jj] = j < i ? Bs[i] * e * kk[u][jj] : 0.f;
          pv[jj] = e * qk[u][jj];
        }
        *reinterpret_cast<float4*>(Am + tri_pad(i, j0)) = float4{av[0], av[1], av[2], av[3]};
        uint2 ph, pl;
        split2(pv[0], pv[1], ph.x, pl.x);
        split2(pv[2], pv[3], ph.y, pl.y);
        const int at = tri_off(i, j0);
        *reinterpret_cast<uint2*>(Pp + at) = ph;
        *reinterpret_cast<uint2*>(Pp + kTri + at) = pl;
      }
    }
    __syncthreads();
    // P, hi and lo, to the tile: the packed bytes as they are, 16 bytes per thread and step.
    for (int u = tid; u < 2 * kTri / 8; u += kThreads)
      *reinterpret_cast<uint4*>(tile->p[0] + 8 * u) = *reinterpret_cast<const uint4*>(Pp + 8 * u);

    // Diagonal blocks: thread -> column j of block bd; the column lives in registers through the substitution.
    if (tid < kC) {
      const int bd = tid >> 4, jl = tid & 15, b0 = 16 * bd;
      float x[16];
#pragma unroll
      for (int il = 0; il < 16; ++il) {
        float v = il == jl ? 1.f : 0.f;
#pragma unroll
        for (int kl = 0; kl < il; ++kl) v -= Am[tri_pad(b0 + il, b0 + kl)] * x[kl];  // x[kl] = 0 for kl < jl
        x[il] = il >= jl ? v : 0.f;
      }
#pragma unroll
      for (int il = 0; il < 16; ++il) Tm[tri_pad(b0 + il, b0 + jl)] = x[il];
    }
    __syncthreads();
    // Off-diagonal blocks at distance d = I - J, one wave per block (wave w: I = d + w, J = w), on MFMA with split
    // float32 operands:
    //   W = sum_{J <= K < I} A_IK T_KJ    16 x 16 x 16d, k zero-padded to a multiple of 32
    //   T_IJ = -T_II W                    16 x 16 x 16, with W's result tile as the B operand (k = W's rows)
    for (int d = 1; d < 4; ++d) {
      if (w < 4 - d) {
        const int I = d + w, J = w;
        f32x4 W = zero4();
        for (int s = 0; s < (d + 1) / 2; ++s) {
          const int k0 = 16 * J + 32 * s + 8 * g;
          const bool in = k0 < 16 * I;  // whole groups of 8 columns are in or out
          float x[8], y[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            x[j] = in ? Am[tri_pad(16 * I + li, k0 + j)] : 0.f;  // A rows 16 I + li, columns k
            y[j] = in ? Tm[tri_pad(k0 + j, 16 * J + li)] : 0.f;  // T rows k, column 16 J + li
          }
          W = mma3(W, split8(x), split8(y));
        }
        uint2 th, tl, wh, wl;  // T_II rows li, k = 4g + j, and W, as packed hi / lo pairs
        {
          const int r = 16 * I + li, c = 16 * I + 4 * g;
          split2(Tm[tri_pad(r, c)], Tm[tri_pad(r, c + 1)], th.x, tl.x);
          split2(Tm[tri_pad(r, c + 2)], Tm[tri_pad(r, c + 3)], th.y, tl.y);
          split2(W[0], W[1], wh.x, wl.x);
          split2(W[2], W[3], wh.y, wl.y);
        }
        f32x4 R = zero4();
        const auto v4 = [](uint2 x) { return __builtin_bit_cast(s16x4, x); };
        R = mma16(R, v4(th), v4(wh));
        R = mma16(R, v4(th), v4(wl));
        R = mma16(R, v4(tl), v4(wh));
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) Tm[tri_pad(16 * I + 4 * g + jj, 16 * J + li)] = -R[jj];
      }
      __syncthreads();
    }

    // T, hi and lo, on and below the diagonal blocks: thread -> row tid / 4, columns 16 (tid % 4) .. + 15.
    {
      const int i = tid >> 2, j0 = (tid & 3) * 16;
      if ((j0 >> 4) <= (i >> 4)) {
        uint32_t th[8], tl[8];  // packed bf16 pairs, columns j0 + 2p, j0 + 2p + 1
#pragma unroll
        for (int p2 = 0; p2 < 8; ++p2) {
          const int j = j0 + 2 * p2;
          split2(Tm[tri_pad(i, j)], Tm[tri_pad(i, j + 1)], th[p2], tl[p2]);
        }
        const int at = tri_off(i, j0);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int q = 4 * h;
          *reinterpret_cast<uint4*>(tile->t[0] + at + 8 * h) = uint4{th[q], th[q + 1], th[q + 2], th[q + 3]};
          *reinterpret_cast<uint4*>(tile->t[1] + at + 8 * h) = uint4{tl[q], tl[q + 1], tl[q + 2], tl[q + 3]};
        }
      }
    }
  }
}

}  // namespace

hipError_t launch_chunk_prep(const ChunkArgs& a, hipStream_t s, bool fused_prologue) {
  if (a.lay.NC == 0) return hipSuccess;
  // One block per (chunk slot, value head) while those blocks fit on the device at once (four per CU: 37 KB of LDS
  // and at most 128 registers each), so that a short sequence's heads run side by side; past that, one per (chunk
  // slot, key head), which reads the group's k and q rows and forms K K^T and Q K^T once for all its value heads and
  // needs half (or a third) of the rounds.
  int dev = 0, cus = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess) return e;
  const int hpb = int64_t(a.lay.NC) * a.Hv <= int64_t(4) * cus ? 1 : a.Hv / a.Hk;
  const dim3 grid(int(a.lay.NC) * (a.Hv / hpb));
  if (fused_prologue)
    hipLaunchKernelGGL(chunk_prep_kernel<true>, grid, dim3(kThreads), 0, s, a, hpb);
  else
    hipLaunchKernelGGL(chunk_prep_kernel<false>, grid, dim3(kThreads), 0, s, a, hpb);
  return hipGetLastError();
}

}  // namespace qbgdn
