// Design 1: the recurrent form. Rows of the state S [Dv, Dk] evolve independently (reference
// src/delta_grad.cpp:13-18), so each row is owned by LPR lanes of a wave, each lane holding NPT = Dk / LPR columns in
// VGPRs for all T steps: LPR = 16 (one DPP row) for Dk up to 96, LPR = 32 from Dk = 128 to 256, so a lane never
// holds more than 8 columns. The two mat-vecs per step are LPR-lane reductions (DPP within 16 lanes, one lane swap
// across two). A block holds the state rows of one value head: 16 rows up to Dk = 128 (4 waves of LPR = 16, or at
// Dk = 128 8 waves of LPR = 32, two waves per SIMD), 8 rows past it (4 waves). The chunk's keys, queries and scalars
// are staged in LDS once per 64 steps and read by all its rows (the backward past Dk = 128 reads the queries from
// global memory instead, to stay within LDS).
//
// Forward (per row, per step), the same recurrence as reference tests/gated_delta_ref.h:46-67 but with both dot
// products taken on the previous state, so one reduction latency per step sits on the dependency chain:
//   a = S_prev k, b = S_prev q;  u = g a;  delta = beta (v - u);  y = g b + delta (k.q);  S = g S_prev + delta k^T
// The chunk-start states (the reference's ckpt, src/delta_grad.cpp:172-181) are written as the forward passes them.
// A call of one token per sequence that keeps neither checkpoints nor per-token states (decode) runs the same step
// in rec_step_kernel, which reads its inputs straight into registers instead of staging a chunk.
//
// The forward also keeps e = v - u per token and state row after the checkpoints in ckpt (4 bytes per token and row).
//
// Backward: reference src/delta_grad.cpp:23-145 re-derived for this layout. Per chunk in reverse: pass A replays
// the chunk's states from its checkpoint with the forward's e (delta = beta e, as the forward formed it), so without
// a reduction, keeping the state at every 8th step in registers; pass B re-forms 8 states at a time from those and
// runs the reverse steps. dq and dk sum over rows: over a wave's rows with lane shuffles, over the block's 4 waves in LDS, over the
// row blocks and the GQA group in rec_reduce_kernel, always in the same order (no atomics).
#include <type_traits>

#include "gdn_common.h"
#include "gdn_kernels.h"

namespace qbgdn {
namespace {

constexpr int kSub = 8;  // states re-formed at a time in the backward
constexpr int kNSub = kChunk / kSub;

// The lane layout for a key width: LPR lanes per state row, NPT columns per lane, waves and rows per block. Dk = 128
// takes LPR = 32 in 8-wave blocks: two waves per SIMD at one block per CU, to hide each other's reduction latency
// (16 rows per block, as with 4 waves of LPR = 16). The wider keys stay at 4 waves for LDS.
template <int NPT, int LPR>
struct Layout {
  static constexpr int kDk = NPT * LPR;
  static constexpr int kWaves = (LPR == 32 && kDk <= 128) ? 8 : 4;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kRowsPerWave = 64 / LPR;
  static constexpr int kRows = kWaves * kRowsPerWave;
};
// Rows per block for a key width (the host side's view of the same layout, and the row-block granularity of the
// backward's partials): 16 up to Dk = 128, 8 up to 256, then the wide kernels' (rec_wide.hip).
inline int rec_rows(int Dk) { return Dk <= 128 ? 16 : Dk <= 256 ? 8 : rec_wide_bwd_rows(Dk); }

// Sum over each group of LPR lanes; every lane of the group gets the same bits.
template <int LPR>
__device__ __forceinline__ float sum_lanes(float x) {
  x = sum16(x);
  if constexpr (LPR == 32) x = swap16_sum(x);
  return x;
}

// The state column of lane cl's i-th value. With NPT a multiple of 4 a lane holds runs of four columns, the LPR
// lanes of a row side by side in each run: a 16-byte LDS read of a step's k or q row by the row's lanes then covers
// every bank once (a lane's NPT contiguous columns would put lanes 8 apart on the same banks). Otherwise a lane
// holds NPT contiguous columns.
template <int NPT, int LPR>
__device__ __forceinline__ int col_of(int cl, int i) {
  if constexpr (NPT % 4 == 0) return (i >> 2) * (4 * LPR) + 4 * cl + (i & 3);
  return cl * NPT + i;
}

struct RecFwdArgs {
  FwdPtrs p;
  float* e_res;  // v - u per token and state row [tokens, Hv, Dv], after the states in ckpt (null without ckpt)
  int Hk, Hv, Dv, g_is_log, nblk, total;
  SeqTable tab;
};

struct RecBwdArgs {
  BwdPtrs p;
  const float* e_res;  // the forward's v - u per token and state row
  int Hk, Hv, Dv, g_is_log, nblk, total;
  float* dq_part;  // [BT, Hv, nblk, Dk]
  float* dk_part;
  float* dg_part;  // [BT, Hv, nblk]
  float* db_part;
  SeqTable tab;
};

// Work item -> (row block, value head, sequence), placed by state_item.
struct Item {
  int blk, hv, n;
};
__device__ __forceinline__ Item item_of(const SeqTable& tab, int nblk, int Hv, int Hk, int total) {
  const StateItem it = state_item(tab, blockIdx.x, nblk, Hv, Hk, total);
  return Item{it.blk, it.hv, it.n};
}

// The staging of a chunk's steps [0, L). With kPad, the steps [L, 64) past a sequence's end are staged as identity
// steps (zero k, q, dy and e, decay factor 1, beta 0), which leave the state and its cotangent unchanged bit for bit,
// so the backward's unrolled steps need no check of their own.

// Stages rows [t0, t0 + L) of the key head's k (and q, when Qs is not null) into LDS as float32, 8 elements per
// access.
template <int kThr, bool kPad = false, int Dk, typename InT>
__device__ __forceinline__ void stage_kq(float (*Ks)[Dk], float (*Qs)[Dk], const InT* k, const InT* q,
                                         int64_t tok, int Hk, int hk, int L) {
  constexpr int V8 = Dk / 8;
  for (int e = threadIdx.x; e < kChunk * V8; e += kThr) {
    const int tt = e / V8, c8 = (e % V8) * 8;
    if (tt < L) {
      const int64_t off = ((tok + tt) * Hk + hk) * Dk + c8;
      IO<InT>::ld8(k + off, &Ks[tt][c8]);
      if (Qs) IO<InT>::ld8(q + off, &Qs[tt][c8]);
    } else if (kPad) {
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        Ks[tt][c8 + u] = 0.f;
        if (Qs) Qs[tt][c8 + u] = 0.f;
      }
    }
  }
}

// Stages a [T, Hv, Dv] tensor's kRows-row slice of rows [t0, t0 + L) (zeros past Dv).
template <int kThr, bool kPad = false, int kRows, typename InT>
__device__ __forceinline__ void stage_rows(float (*Xs)[kRows], const InT* x, int64_t tok, int Hv, int hv, int Dv,
                                           int row0, int L) {
  for (int e = threadIdx.x; e < kChunk * kRows; e += kThr) {
    const int tt = e / kRows, j = e % kRows;
    if (tt < L)
      Xs[tt][j] = (row0 + j < Dv) ? IO<InT>::ld(x, ((tok + tt) * Hv + hv) * Dv + row0 + j) : 0.f;
    else if (kPad)
      Xs[tt][j] = 0.f;
  }
}

// Per-step scalars: the decay factor (exp of the log-decay when g_is_log) and beta, as the first two of W floats
// per step (the step's scalars are read together, one vector read at a uniform address).
template <int kThr, bool kPad = false, int W, typename InT>
__device__ __forceinline__ void stage_scalars(float (*GB)[W], const float* g, const InT* beta, int64_t tok, int Hv,
                                              int hv, int L, int g_is_log) {
  for (int tt = threadIdx.x; tt < (kPad ? kChunk : L); tt += kThr) {
    if (tt < L) {
      const int64_t i = (tok + tt) * Hv + hv;
      const float gv = g[i];
      GB[tt][0] = g_is_log ? expf(gv) : gv;
      GB[tt][1] = IO<InT>::ld(beta, i);
    } else {
      GB[tt][0] = 1.f, GB[tt][1] = 0.f;
    }
  }
}

// kKeepRows: also store the state after every token (a.p.rows), for the per-token-state forward.
template <int NPT, int LPR, typename InT, typename OutT, bool kKeepRows>
__global__ __launch_bounds__((Layout<NPT, LPR>::kThreads)) void rec_fwd_kernel(RecFwdArgs a) {
  using Lay = Layout<NPT, LPR>;
  constexpr int Dk = LPR * NPT, kRows = Lay::kRows, kThreads = Lay::kThreads;
  // One LDS array, the small per-step arrays first: at low addresses every access to them takes an immediate offset
  // from one base register (a ds_read reaches 64 KB past its address) instead of a materialized address per step.
  constexpr int oGBK = 0, oV = oGBK + kChunk * 4 * 4, oYE = oV + kChunk * kRows * 4, oK = oYE + kChunk * kRows * 8;
  constexpr int oQ = oK + kChunk * Dk * 4, kLdsBytes = oQ + kChunk * Dk * 4;
  __shared__ __align__(16) unsigned char lds[kLdsBytes];
  auto GBK = reinterpret_cast<float (*)[4]>(lds + oGBK);  // per step: decay factor, beta, k.q
  auto Vs = reinterpret_cast<float (*)[kRows]>(lds + oV);
  auto YEs = reinterpret_cast<float2 (*)[kRows]>(lds + oYE);  // y and e = v - u per step and row
  auto Ks = reinterpret_cast<float (*)[Dk]>(lds + oK);
  auto Qs = reinterpret_cast<float (*)[Dk]>(lds + oQ);

  const Item it = item_of(a.tab, a.nblk, a.Hv, a.Hk, a.total);
  const int tid = threadIdx.x, lane = tid & 63;
  const int cl = lane % LPR, rl = (tid >> 6) * Lay::kRowsPerWave + lane / LPR;
  const int row0 = it.blk * kRows, row = row0 + rl;
  const bool live = row < a.Dv;
  const int hv = it.hv, hk = hv / (a.Hv / a.Hk);
  const Seq sq = seq_of(a.tab, it.n);
  const InT* q = static_cast<const InT*>(a.p.q);
  const InT* k = static_cast<const InT*>(a.p.k);
  const InT* v = static_cast<const InT*>(a.p.v);
  const InT* beta = static_cast<const InT*>(a.p.beta);
  OutT* y = static_cast<OutT*>(a.p.y);
  const int64_t SS = int64_t(a.Dv) * Dk;
  const int64_t srow = (int64_t(it.n) * a.Hv + hv) * SS + int64_t(row) * Dk;  // the row's first column

  float s[NPT];
#pragma unroll
  for (int i = 0; i < NPT; ++i) s[i] = (live && a.p.s0) ? a.p.s0[srow + col_of<NPT, LPR>(cl, i)] : 0.f;

  const int nch = (sq.len + kChunk - 1) / kChunk;
  for (int c = 0; c < nch; ++c) {
    const int t0 = c * kChunk, L = min(kChunk, sq.len - t0);
    const int64_t tok = sq.tok0 + t0;
    if (a.p.ckpt && live) {
      float* dst = a.p.ckpt + ((sq.slot0 + c) * a.Hv + hv) * SS + int64_t(row) * Dk;
#pragma unroll
      for (int i = 0; i < NPT; ++i) dst[col_of<NPT, LPR>(cl, i)] = s[i];
    }
    __syncthreads();  // the previous chunk's LDS readers are done
    stage_kq<kThreads>(Ks, Qs, (const InT*)k, (const InT*)q, tok, a.Hk, hk, L);
    stage_rows<kThreads>(Vs, v, tok, a.Hv, hv, a.Dv, row0, L);
    stage_scalars<kThreads>(GBK, a.p.g, beta, tok, a.Hv, hv, L, a.g_is_log);
    __syncthreads();
    // k.q per step: groups of LPR lanes, one step each at a time.
    for (int tt = tid / LPR; tt < kChunk; tt += kThreads / LPR) {
      float kq = 0.f;
#pragma unroll
      for (int i = 0; i < NPT; ++i) kq += Ks[tt][col_of<NPT, LPR>(cl, i)] * Qs[tt][col_of<NPT, LPR>(cl, i)];
      kq = sum_lanes<LPR>(kq);
      if (cl == 0) GBK[tt][2] = kq;
    }
    __syncthreads();
    auto step = [&](const int tt) {
      float kk[NPT], qq[NPT];
#pragma unroll
      for (int i = 0; i < NPT; ++i) kk[i] = Ks[tt][col_of<NPT, LPR>(cl, i)], qq[i] = Qs[tt][col_of<NPT, LPR>(cl, i)];
      float pa = 0.f, pb = 0.f;
#pragma unroll
      for (int i = 0; i < NPT; ++i) pa = fmaf(s[i], kk[i], pa), pb = fmaf(s[i], qq[i], pb);
      if constexpr (LPR == 32) {
        sum32_pair(pa, pb);
      } else {
        pa = sum_lanes<LPR>(pa);
        pb = sum_lanes<LPR>(pb);
      }
      // Each rounding written out (fmaf), so that both copies of the step below, in every variant of the kernel,
      // form the same bits: a multi-token call and one-token calls from its per-token states agree exactly.
      const float4 gbk = *reinterpret_cast<const float4*>(GBK[tt]);
      const float gt = gbk.x, bt = gbk.y;
      const float e = fmaf(-gt, pa, Vs[tt][rl]);
      const float d = bt * e;
      const float yv = fmaf(gt, pb, d * gbk.z);
#pragma unroll
      for (int i = 0; i < NPT; ++i) s[i] = fmaf(gt, s[i], d * kk[i]);
      YEs[tt][rl] = float2{yv, e};  // every lane of the row holds the same bits: a store without a branch
      if (kKeepRows && live) {  // the state after this token
        float* dst = a.p.rows + ((tok + tt) * a.Hv + hv) * SS + int64_t(row) * Dk;
#pragma unroll
        for (int i = 0; i < NPT; ++i) dst[col_of<NPT, LPR>(cl, i)] = s[i];
      }
    };
    // Steps in pairs, written out (the compiler does not unroll a loop of lane swaps with a run-time count), so that
    // the two copies alternate their registers instead of copying the state at every step.
    int tt = 0;
    for (; tt + 1 < L; tt += 2) {
      step(tt);
      step(tt + 1);
    }
    if (tt < L) step(tt);
    __syncthreads();
    for (int e = tid; e < L * kRows; e += kThreads) {
      const int tt = e / kRows, j = e % kRows;
      if (row0 + j < a.Dv) {
        const int64_t at = ((tok + tt) * a.Hv + hv) * a.Dv + row0 + j;
        const float2 ye = YEs[tt][j];
        IO<OutT>::st(y, at, ye.x);
        if (a.e_res) a.e_res[at] = ye.y;
      }
    }
  }
  if (a.p.s_out && live) {
#pragma unroll
    for (int i = 0; i < NPT; ++i) a.p.s_out[srow + col_of<NPT, LPR>(cl, i)] = s[i];
  }
}

// The one-token step (decode, reference src/deltanet.cpp:101-120): every sequence of the call has at most one token,
// and neither checkpoints nor per-token states are asked for. The same work items, lanes and arithmetic as
// rec_fwd_kernel's step, so the same bits, but every input goes straight from memory into the registers of the lanes
// that use it (a lane's k and q columns, its row's v, the head's decay factor and beta), issued together with the
// state's loads: no LDS staging, no barrier, and one memory round trip before the step.
template <int NPT, int LPR, typename InT, typename OutT>
__global__ __launch_bounds__((Layout<NPT, LPR>::kThreads)) void rec_step_kernel(RecFwdArgs a) {
  using Lay = Layout<NPT, LPR>;
  constexpr int Dk = LPR * NPT;
  const Item it = item_of(a.tab, a.nblk, a.Hv, a.Hk, a.total);
  const int tid = threadIdx.x, lane = tid & 63;
  const int cl = lane % LPR, rl = (tid >> 6) * Lay::kRowsPerWave + lane / LPR;
  const int row = it.blk * Lay::kRows + rl;
  const bool live = row < a.Dv;
  const int hv = it.hv, hk = hv / (a.Hv / a.Hk);
  const Seq sq = seq_of(a.tab, it.n);
  const int64_t SS = int64_t(a.Dv) * Dk;
  const int64_t srow = (int64_t(it.n) * a.Hv + hv) * SS + int64_t(row) * Dk;

  float s[NPT];
#pragma unroll
  for (int i = 0; i < NPT; ++i) s[i] = (live && a.p.s0) ? a.p.s0[srow + col_of<NPT, LPR>(cl, i)] : 0.f;
  if (sq.len > 0) {  // uniform over the block; an empty sequence keeps its state
    const InT* q = static_cast<const InT*>(a.p.q);
    const InT* k = static_cast<const InT*>(a.p.k);
    const InT* v = static_cast<const InT*>(a.p.v);
    const int64_t kb = (sq.tok0 * a.Hk + hk) * Dk, hb = sq.tok0 * a.Hv + hv;
    float kk[NPT], qq[NPT];
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      kk[i] = IO<InT>::ld(k, kb + col_of<NPT, LPR>(cl, i));
      qq[i] = IO<InT>::ld(q, kb + col_of<NPT, LPR>(cl, i));
    }
    const float gv = a.p.g[hb];
    const float gt = a.g_is_log ? expf(gv) : gv;
    const float bt = IO<InT>::ld(static_cast<const InT*>(a.p.beta), hb);
    const float vv = live ? IO<InT>::ld(v, hb * a.Dv + row) : 0.f;
    float kq = 0.f;
#pragma unroll
    for (int i = 0; i < NPT; ++i) kq += kk[i] * qq[i];
    kq = sum_lanes<LPR>(kq);
    float pa = 0.f, pb = 0.f;
#pragma unroll
    for (int i = 0; i < NPT; ++i) pa = fmaf(s[i], kk[i], pa), pb = fmaf(s[i], qq[i], pb);
    if constexpr (LPR == 32) {
      sum32_pair(pa, pb);
    } else {
      pa = sum_lanes<LPR>(pa);
      pb = sum_lanes<LPR>(pb);
    }
    const float e = fmaf(-gt, pa, vv);
    const float d = bt * e;
    const float yv = fmaf(gt, pb, d * kq);
#pragma unroll
    for (int i = 0; i < NPT; ++i) s[i] = fmaf(gt, s[i], d * kk[i]);
    if (live && cl == 0) IO<OutT>::st(static_cast<OutT*>(a.p.y), hb * a.Dv + row, yv);
  }
  if (a.p.s_out && live) {
#pragma unroll
    for (int i = 0; i < NPT; ++i) a.p.s_out[srow + col_of<NPT, LPR>(cl, i)] = s[i];
  }
}

// Sums NPT per-lane column values over the wave's rows and writes each column's sum once into dst[0, Dk). LPR = 16:
// lanes l, l^16, l^32, l^48 hold the same columns of the wave's 4 rows; with NPT a multiple of 4 the values are
// halved at each exchange so each lane ends with NPT/4 finished columns, otherwise a plain butterfly is used. LPR = 32:
// lanes l and l^32 hold the same columns of the wave's 2 rows.
template <int NPT, int LPR>
__device__ __forceinline__ void wave_rows_sum(const float* p, float* dst, int lane) {
  const int cl = lane % LPR;
  if constexpr (LPR == 16 && NPT % 4 == 0) {
    constexpr int H = NPT / 2, Q = NPT / 4;
    const bool h32 = lane & 32, h16 = lane & 16;
    // Each exchange is one gfx950 lane swap (VALU, no LDS): v_permlane32_swap(a, b) leaves (a, a of lane + 32) in
    // lanes 0-31 and (b of lane - 32, b) in lanes 32-63, so the sum of its two results is, in every lane, the lane's
    // kept value plus its partner's sent one; v_permlane16_swap does the same between the 16-lane halves of each 32.
    float w[H], x[Q];
#pragma unroll
    for (int j = 0; j < H; ++j) {
      const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(p[j]), __float_as_uint(p[j + H]), false, false);
      w[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
#pragma unroll
    for (int j = 0; j < Q; ++j) {
      const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(w[j]), __float_as_uint(w[j + Q]), false, false);
      x[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    const int i0 = (h16 ? Q : 0) + (h32 ? H : 0);  // the lane's finished values: i0 .. i0 + Q - 1
#pragma unroll
    for (int j = 0; j < Q; ++j) dst[col_of<NPT, LPR>(cl, i0 + j)] = x[j];
  } else if constexpr (LPR == 32 && NPT % 2 == 0) {
    constexpr int H = NPT / 2;
    float w[H];
#pragma unroll
    for (int j = 0; j < H; ++j) {
      const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(p[j]), __float_as_uint(p[j + H]), false, false);
      w[j] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    const int i0 = lane & 32 ? H : 0;
#pragma unroll
    for (int j = 0; j < H; ++j) dst[col_of<NPT, LPR>(cl, i0 + j)] = w[j];
  } else {
#pragma unroll
    for (int j = 0; j < NPT; ++j) {
      float x = swap32_sum(p[j]);
      if constexpr (LPR == 16) x = swap16_sum(x);
      if (lane < LPR) dst[col_of<NPT, LPR>(cl, j)] = x;
    }
  }
}

// The wide variant (LPR = 32) reads q from global memory in its reverse steps rather than staging it: its k, red and
// the per-row arrays take about 137 KB of LDS at Dk = 256.
template <int NPT, int LPR, typename InT, typename OutT>
__global__ __launch_bounds__((Layout<NPT, LPR>::kThreads)) void rec_bwd_kernel(RecBwdArgs a) {
  using Lay = Layout<NPT, LPR>;
  constexpr int Dk = LPR * NPT, kRows = Lay::kRows, kThreads = Lay::kThreads, kWaves = Lay::kWaves;
  constexpr bool kQGlobal = Dk > 128;
  // Steps past a sequence's end staged as identity steps (the stage_ helpers), so the unrolled steps run unchecked;
  // not with kQGlobal, whose reverse steps read q from global memory, where such a step has no row.
  constexpr bool kPad = !kQGlobal;
  // One LDS array, the small per-step arrays first (low addresses: immediate offsets from one base register).
  constexpr int oGB = 0, oDY = oGB + kChunk * 2 * 4, oE = oDY + kChunk * kRows * 4, oRow = oE + kChunk * kRows * 4;
  constexpr int oRed = (oRow + kSub * 3 * kRows * 4 + 15) / 16 * 16, oK = oRed + kSub * kWaves * 2 * Dk * 4;
  constexpr int oQ = oK + kChunk * Dk * 4, kLdsBytes = oQ + (kQGlobal ? 1 : kChunk) * Dk * 4;
  __shared__ __align__(16) unsigned char lds[kLdsBytes];
  auto GB = reinterpret_cast<float (*)[2]>(lds + oGB);  // per step: decay factor, beta
  auto DYs = reinterpret_cast<float (*)[kRows]>(lds + oDY);
  auto Es = reinterpret_cast<float (*)[kRows]>(lds + oE);
  auto rowv = reinterpret_cast<float (*)[3][kRows]>(lds + oRow);  // per step and row: dv, dbeta, dg (factor)
  // per step and wave: column sums of (dq | dk) over the wave's rows
  auto red = reinterpret_cast<float (*)[kWaves][2 * Dk]>(lds + oRed);
  auto Ks = reinterpret_cast<float (*)[Dk]>(lds + oK);
  auto Qs = reinterpret_cast<float (*)[Dk]>(lds + oQ);

  const Item it = item_of(a.tab, a.nblk, a.Hv, a.Hk, a.total);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int cl = lane % LPR, rl = wave * Lay::kRowsPerWave + lane / LPR;
  const int row0 = it.blk * kRows, row = row0 + rl;
  const bool live = row < a.Dv;
  const int hv = it.hv, hk = hv / (a.Hv / a.Hk);
  const Seq sq = seq_of(a.tab, it.n);
  const InT* q = static_cast<const InT*>(a.p.q);
  const InT* k = static_cast<const InT*>(a.p.k);
  const OutT* dy = static_cast<const OutT*>(a.p.dy);
  const InT* beta = static_cast<const InT*>(a.p.beta);
  OutT* dv = static_cast<OutT*>(a.p.dv);
  const int64_t SS = int64_t(a.Dv) * Dk;
  const int64_t srow = (int64_t(it.n) * a.Hv + hv) * SS + int64_t(row) * Dk;  // the row's first column

  float ds[NPT];
#pragma unroll
  for (int i = 0; i < NPT; ++i) ds[i] = (live && a.p.ds_out) ? a.p.ds_out[srow + col_of<NPT, LPR>(cl, i)] : 0.f;

  const int nch = (sq.len + kChunk - 1) / kChunk;
  for (int c = nch - 1; c >= 0; --c) {
    const int t0 = c * kChunk, L = min(kChunk, sq.len - t0);
    const int64_t tok = sq.tok0 + t0;
    __syncthreads();
    stage_kq<kThreads, kPad>(Ks, kQGlobal ? nullptr : Qs, k, q, tok, a.Hk, hk, L);
    stage_rows<kThreads, kPad>(Es, a.e_res, tok, a.Hv, hv, a.Dv, row0, L);
    stage_rows<kThreads, kPad>(DYs, dy, tok, a.Hv, hv, a.Dv, row0, L);
    stage_scalars<kThreads, kPad>(GB, a.p.g, beta, tok, a.Hv, hv, L, a.g_is_log);
    float st[NPT];
    {
      const float* src = a.p.ckpt + ((sq.slot0 + c) * a.Hv + hv) * SS + int64_t(row) * Dk;
#pragma unroll
      for (int i = 0; i < NPT; ++i) st[i] = live ? src[col_of<NPT, LPR>(cl, i)] : 0.f;
    }
    __syncthreads();

    // Pass A: replay the chunk's states (delta = beta e, the forward's product), keeping every kSub-th one.
    float sub[kNSub][NPT];
    for (int m = 0; m < kNSub; ++m) {
#pragma unroll
      for (int mm = 0; mm < kNSub; ++mm)
        if (mm == m) {
#pragma unroll
          for (int i = 0; i < NPT; ++i) sub[mm][i] = st[i];
        }
#pragma unroll
      for (int j = 0; j < kSub; ++j) {
        const int tt = m * kSub + j;
        if (kPad || tt < L) {
          const float2 gb = *reinterpret_cast<const float2*>(GB[tt]);
          const float gt = gb.x, d = gb.y * Es[tt][rl];
#pragma unroll
          for (int i = 0; i < NPT; ++i) st[i] = gt * st[i] + d * Ks[tt][col_of<NPT, LPR>(cl, i)];
        }
      }
    }

    // Pass B: 8 states at a time from the kept starts, then the reverse steps (reference :97-141).
    for (int m = kNSub - 1; m >= 0; --m) {
      const int ts = m * kSub;
      if (ts >= L) continue;  // uniform over the block
      float S[kSub + 1][NPT];
#pragma unroll
      for (int i = 0; i < NPT; ++i) S[0][i] = 0.f;
#pragma unroll
      for (int mm = 0; mm < kNSub; ++mm)
        if (mm == m) {
#pragma unroll
          for (int i = 0; i < NPT; ++i) S[0][i] = sub[mm][i];
        }
#pragma unroll
      for (int j = 0; j < kSub; ++j) {
        const int tt = ts + j;
        if (kPad || tt < L) {
          const float2 gb = *reinterpret_cast<const float2*>(GB[tt]);
          const float gt = gb.x, d = gb.y * Es[tt][rl];
#pragma unroll
          for (int i = 0; i < NPT; ++i) S[j + 1][i] = gt * S[j][i] + d * Ks[tt][col_of<NPT, LPR>(cl, i)];
        } else {
#pragma unroll
          for (int i = 0; i < NPT; ++i) S[j + 1][i] = S[j][i];
        }
      }
      // With LPR = 32, a step's dg is summed over the row's lanes together with the next (lower) step's dd, one
      // paired reduction for the two (dgp holds it meanwhile).
      float dgp = 0.f;
#pragma unroll
      for (int j = kSub - 1; j >= 0; --j) {
        const int tt = ts + j;
        if (!kPad && tt >= L) continue;
        float kk[NPT], qq[NPT], pq[NPT], pk[NPT];
#pragma unroll
        for (int i = 0; i < NPT; ++i) {
          kk[i] = Ks[tt][col_of<NPT, LPR>(cl, i)];
          qq[i] = kQGlobal ? IO<InT>::ld(q, ((tok + tt) * a.Hk + hk) * Dk + col_of<NPT, LPR>(cl, i)) : Qs[tt][col_of<NPT, LPR>(cl, i)];
        }
        const float2 gb = *reinterpret_cast<const float2*>(GB[tt]);
        const float gt = gb.x, bt = gb.y, dyt = DYs[tt][rl], e = Es[tt][rl], d = bt * e;
        float dd = 0.f;
#pragma unroll
        for (int i = 0; i < NPT; ++i) {
          ds[i] += dyt * qq[i];
          pq[i] = dyt * S[j + 1][i];
          dd += ds[i] * kk[i];
        }
        if constexpr (LPR == 32) {
          if (j < kSub - 1) {
            sum32_pair(dd, dgp);
            rowv[j + 1][2][rl] = dgp;  // step j + 1's dg (not read past the sub-chunk's last step)
          } else {
            dd = sum_lanes<LPR>(dd);
          }
        } else {
          dd = sum_lanes<LPR>(dd);
        }
        const float du = -bt * dd, dug = du * gt;
        float dg = 0.f;
#pragma unroll
        for (int i = 0; i < NPT; ++i) {
          pk[i] = ds[i] * d + dug * S[j][i];
          ds[i] += du * kk[i];
          dg += ds[i] * S[j][i];
          ds[i] *= gt;
        }
        if constexpr (LPR == 32) {
          dgp = dg;
        } else {
          dg = sum_lanes<LPR>(dg);
          rowv[j][2][rl] = dg;
        }
        rowv[j][0][rl] = bt * dd, rowv[j][1][rl] = dd * e;  // row-uniform, every lane
        wave_rows_sum<NPT, LPR>(pq, red[j][wave], lane);
        wave_rows_sum<NPT, LPR>(pk, red[j][wave] + Dk, lane);
      }
      if constexpr (LPR == 32) rowv[0][2][rl] = sum_lanes<LPR>(dgp);  // the sub-chunk's first step (always run)
      __syncthreads();
      const int Ls = min(kSub, L - ts);
      // Four columns per thread and pass (16-byte reads and stores), a fixed trip count, unrolled, so that every
      // pass's LDS reads issue together rather than one round trip per pass; passes past the sub-chunk's last step
      // store nothing. The waves' sums add in wave order.
      constexpr int kU = Dk / 2;  // 4-column units of a step's (dq | dk) row
      constexpr int kPasses = (kSub * kU + kThreads - 1) / kThreads;
#pragma unroll
      for (int pss = 0; pss < kPasses; ++pss) {
        const int e = tid + pss * kThreads;
        if (e < Ls * kU) {
          const int j = e / kU, col = (e % kU) * 4;
          float4 acc = *reinterpret_cast<const float4*>(&red[j][0][col]);
#pragma unroll
          for (int w = 1; w < kWaves; ++w) {
            const float4 x = *reinterpret_cast<const float4*>(&red[j][w][col]);
            acc.x += x.x, acc.y += x.y, acc.z += x.z, acc.w += x.w;
          }
          const int64_t at = (((tok + ts + j) * a.Hv + hv) * a.nblk + it.blk) * Dk;
          float* dst = col < Dk ? a.dq_part + at + col : a.dk_part + at + col - Dk;
          // Written once and read once by the reduction: streaming stores.
          typedef float v4f __attribute__((ext_vector_type(4)));
          __builtin_nontemporal_store(v4f{acc.x, acc.y, acc.z, acc.w}, reinterpret_cast<v4f*>(dst));
        }
      }
      for (int e = tid; e < Ls * kRows; e += kThreads) {
        const int j = e / kRows, r = e % kRows;
        if (row0 + r < a.Dv) IO<OutT>::st(dv, ((tok + ts + j) * a.Hv + hv) * a.Dv + row0 + r, rowv[j][0][r]);
      }
      if (tid < 2 * Ls) {
        const int j = tid >> 1, which = tid & 1;  // 0: dbeta, 1: dg
        float acc = 0.f;
        for (int r = 0; r < kRows; ++r) acc += rowv[j][1 + which][r];
        const int64_t at = ((tok + ts + j) * a.Hv + hv) * a.nblk + it.blk;
        (which ? a.dg_part : a.db_part)[at] = acc;
      }
      __syncthreads();
    }
  }
  if (a.p.ds0 && live) {
#pragma unroll
    for (int i = 0; i < NPT; ++i) a.p.ds0[srow + col_of<NPT, LPR>(cl, i)] = ds[i];
  }
}

// dq, dk [BT, Hk, Dk] = sum over the group's value heads, then over row blocks, of the partials (reference
// src/delta_grad.cpp:194-198 sums row blocks first; both orders are fixed). dg, dbeta [BT, Hv] likewise over row
// blocks; dg becomes d/d(log-decay) when g_is_log.
template <typename OutT>
__global__ __launch_bounds__(256) void rec_reduce_kernel(const float* dq_part, const float* dk_part,
                                                         const float* dg_part, const float* db_part, const float* g,
                                                         OutT* dq, OutT* dk, float* dg, OutT* dbeta, int Hk, int Hv,
                                                         int Dk, int nblk, int g_is_log, int64_t items) {
  // Eight (token, key head) items per block, 32 lanes each, four columns per lane: an item's partials are
  // grp * nblk contiguous rows of Dk floats, read as 16-byte units and summed in row order (value head, then row
  // block), the fixed order of the reference (src/delta_grad.cpp:194-198 over row blocks).
  const int64_t item = int64_t(blockIdx.x) * 8 + (threadIdx.x >> 5);
  if (item >= items) return;
  const int l32 = threadIdx.x & 31;
  const int64_t tok = item / Hk;
  const int hk = int(item % Hk), grp = Hv / Hk, np = grp * nblk;
  const int64_t base = (tok * Hv + int64_t(hk) * grp) * nblk;  // the item's first partial row
  for (int c = 4 * l32; c < Dk; c += 128) {
    float4 aq = {0.f, 0.f, 0.f, 0.f}, ak = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
    for (int pr = 0; pr < np; ++pr) {
      // Read once: streaming loads (the partials are not reused).
      typedef float v4f __attribute__((ext_vector_type(4)));
      const v4f xq = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(dq_part + (base + pr) * Dk + c));
      const v4f xk = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(dk_part + (base + pr) * Dk + c));
      aq.x += xq.x, aq.y += xq.y, aq.z += xq.z, aq.w += xq.w;
      ak.x += xk.x, ak.y += xk.y, ak.z += xk.z, ak.w += xk.w;
    }
    const int64_t o = (tok * Hk + hk) * Dk + c;
    IO<OutT>::st(dq, o, aq.x), IO<OutT>::st(dq, o + 1, aq.y), IO<OutT>::st(dq, o + 2, aq.z);
    IO<OutT>::st(dq, o + 3, aq.w);
    IO<OutT>::st(dk, o, ak.x), IO<OutT>::st(dk, o + 1, ak.y), IO<OutT>::st(dk, o + 2, ak.z);
    IO<OutT>::st(dk, o + 3, ak.w);
  }
  if (l32 < grp) {
    const int hv = hk * grp + l32;
    float ag = 0.f, ab = 0.f;
    for (int b = 0; b < nblk; ++b) {
      ag += dg_part[(tok * Hv + hv) * nblk + b];
      ab += db_part[(tok * Hv + hv) * nblk + b];
    }
    const float gv = g[tok * Hv + hv];
    dg[tok * Hv + hv] = g_is_log ? ag * expf(gv) : ag;
    IO<OutT>::st(dbeta, tok * Hv + hv, ab);
  }
}

// Calls f(NPT, LPR) (as integral constants) for the key widths the kernels are built for: every multiple of 32 up to
// 256. Returns false for any other width.
template <class F>
bool with_width(int Dk, F&& f) {
  using std::integral_constant;
  switch (Dk) {
    case 32: f(integral_constant<int, 2>{}, integral_constant<int, 16>{}); return true;
    case 64: f(integral_constant<int, 4>{}, integral_constant<int, 16>{}); return true;
    case 96: f(integral_constant<int, 6>{}, integral_constant<int, 16>{}); return true;
    case 128: f(integral_constant<int, 4>{}, integral_constant<int, 32>{}); return true;
    case 160: f(integral_constant<int, 5>{}, integral_constant<int, 32>{}); return true;
    case 192: f(integral_constant<int, 6>{}, integral_constant<int, 32>{}); return true;
    case 224: f(integral_constant<int, 7>{}, integral_constant<int, 32>{}); return true;
    case 256: f(integral_constant<int, 8>{}, integral_constant<int, 32>{}); return true;
    default: return false;
  }
}

int row_blocks(const Problem& p) {
  const int rows = rec_rows(p.Dk);
  return (p.Dv + rows - 1) / rows;
}

template <typename InT, typename OutT>
hipError_t launch_fwd(const Problem& p, const FwdPtrs& ptrs, hipStream_t s, Tracer& tr) {
  RecFwdArgs a;
  a.p = ptrs;
  a.e_res = ptrs.ckpt ? ptrs.ckpt + int64_t(p.NC) * p.Hv * p.Dv * p.Dk : nullptr;
  a.Hk = p.Hk, a.Hv = p.Hv, a.Dv = p.Dv, a.g_is_log = p.g_is_log;
  a.nblk = row_blocks(p);
  a.total = a.nblk * p.Hv * p.N;
  a.tab = p.tab;
  const dim3 grid(a.total);
  tr.mark();
  if (p.Dk > 256) {  // one wave per row (rec_wide.hip)
    const hipError_t e = rec_wide_fwd<InT, OutT>(p, ptrs, s);
    tr.mark();
    return e;
  }
  const bool rows = ptrs.rows != nullptr;
  // One token or none per sequence (batch mode with T = 1; packed, where every sequence that is not empty has one
  // chunk slot per token), with nothing to keep but y and the final state: the one-token step.
  const bool one = (p.tab.n == 0 ? p.T <= 1 : p.NC == p.BT) && !ptrs.ckpt && !rows;
  const bool ok = with_width(p.Dk, [&](auto npt, auto lpr) {
    constexpr int NPT = decltype(npt)::value, LPR = decltype(lpr)::value;
    const dim3 block(Layout<NPT, LPR>::kThreads);
    if (one)
      hipLaunchKernelGGL((rec_step_kernel<NPT, LPR, InT, OutT>), grid, block, 0, s, a);
    else if (rows)
      hipLaunchKernelGGL((rec_fwd_kernel<NPT, LPR, InT, OutT, true>), grid, block, 0, s, a);
    else
      hipLaunchKernelGGL((rec_fwd_kernel<NPT, LPR, InT, OutT, false>), grid, block, 0, s, a);
  });
  if (!ok) return hipErrorInvalidValue;
  tr.mark();
  return hipGetLastError();
}

struct BwdWs {
  float *dq_part, *dk_part, *dg_part, *db_part, *scratch;
};

// The partials, then (past Dk = 256) the wide backward's per-row scratch.
BwdWs carve(const Problem& p, void* ws) {
  const int64_t nblk = row_blocks(p);
  const int64_t big = p.BT * p.Hv * nblk * p.Dk, small = p.BT * p.Hv * nblk;
  float* f = static_cast<float*>(ws);
  return BwdWs{f, f + big, f + 2 * big, f + 2 * big + small, f + 2 * big + 2 * small};
}

template <typename InT, typename OutT>
hipError_t launch_bwd(const Problem& p, const BwdPtrs& ptrs, void* ws, hipStream_t s, Tracer& tr) {
  RecBwdArgs a;
  a.p = ptrs;
  a.e_res = ptrs.ckpt + int64_t(p.NC) * p.Hv * p.Dv * p.Dk;
  a.Hk = p.Hk, a.Hv = p.Hv, a.Dv = p.Dv, a.g_is_log = p.g_is_log;
  a.nblk = row_blocks(p);
  a.total = a.nblk * p.Hv * p.N;
  const BwdWs w = carve(p, ws);
  a.dq_part = w.dq_part, a.dk_part = w.dk_part, a.dg_part = w.dg_part, a.db_part = w.db_part;
  a.tab = p.tab;
  const dim3 grid(a.total);
  tr.mark();
  hipError_t e = hipSuccess;
  if (p.Dk > 256) {  // one wave per row (rec_wide.hip)
    e = rec_wide_bwd<InT, OutT>(p, ptrs, w.dq_part, w.dk_part, w.dg_part, w.db_part, w.scratch, a.nblk, s);
  } else {
    const bool ok = with_width(p.Dk, [&](auto npt, auto lpr) {
      constexpr int NPT = decltype(npt)::value, LPR = decltype(lpr)::value;
      const dim3 block(Layout<NPT, LPR>::kThreads);
      hipLaunchKernelGGL((rec_bwd_kernel<NPT, LPR, InT, OutT>), grid, block, 0, s, a);
    });
    if (!ok) return hipErrorInvalidValue;
    e = hipGetLastError();
  }
  if (e != hipSuccess) return e;
  tr.mark();
  if (p.BT == 0) {
    tr.mark();
    return hipSuccess;
  }
  const int64_t items = p.BT * p.Hk;
  hipLaunchKernelGGL((rec_reduce_kernel<OutT>), dim3(static_cast<unsigned>((items + 7) / 8)), dim3(256), 0, s,
                     w.dq_part, w.dk_part, w.dg_part, w.db_part, ptrs.g, static_cast<OutT*>(ptrs.dq),
                     static_cast<OutT*>(ptrs.dk), ptrs.dg, static_cast<OutT*>(ptrs.dbeta), p.Hk, p.Hv, p.Dk, a.nblk,
                     p.g_is_log, items);
  tr.mark();
  return hipGetLastError();
}

}  // namespace

// The reference's vjp takes Dk a multiple of 32 whose 2 * Dk * 4-byte row reduction fits its 32 KB of threadgroup
// memory (src/delta_grad.cpp:159-170), so at most 4096.
const char* rec_supports(const Problem& p) {
  if (p.Dk % 32 || p.Dk > 4096) return "the recurrent design needs Dk a multiple of 32 of at most 4096";
  return nullptr;
}

// The chunk-start states [NC, Hv, Dv, Dk], then e = v - u [tokens, Hv, Dv].
size_t rec_ckpt_bytes(const Problem& p) {
  return (size_t(p.NC) * p.Hv * p.Dv * p.Dk + size_t(p.BT) * p.Hv * p.Dv) * sizeof(float);
}

size_t rec_workspace_bytes(const Problem& p) {
  const size_t nblk = row_blocks(p);
  const size_t parts = (2 * size_t(p.BT) * p.Hv * nblk * p.Dk + 2 * size_t(p.BT) * p.Hv * nblk) * sizeof(float);
  return parts + (p.Dk > 256 ? rec_wide_scratch_bytes(p) : 0);
}

const char* const kRecFwdLaunches = "rec_fwd";
const char* const kRecBwdLaunches = "rec_bwd,rec_reduce";

hipError_t rec_fwd(const Problem& p, const FwdPtrs& a, void*, hipStream_t s, Tracer& tr) {
  if (!p.in_bf16) return launch_fwd<float, float>(p, a, s, tr);
  return p.out_bf16 ? launch_fwd<bf16_t, bf16_t>(p, a, s, tr) : launch_fwd<bf16_t, float>(p, a, s, tr);
}

hipError_t rec_bwd(const Problem& p, const BwdPtrs& a, void* ws, hipStream_t s, Tracer& tr) {
  if (!p.in_bf16) return launch_bwd<float, float>(p, a, ws, s, tr);
  return p.out_bf16 ? launch_bwd<bf16_t, bf16_t>(p, a, ws, s, tr) : launch_bwd<bf16_t, float>(p, a, ws, s, tr);
}

}  // namespace qbgdn
