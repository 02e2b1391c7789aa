// Design 1 past Dk = 256: the recurrent form for every key width the reference's vjp accepts beyond the
// register-resident kernels of rec.hip, multiples of 32 up to 4096 (src/delta_grad.cpp:159-170: Dk % 32, and its
// 2 * Dk * 4-byte row reduction within 32 KB of threadgroup memory). It follows the same per-row recurrence and the
// same backward steps as rec.hip (reference src/delta_grad.cpp:97-141), with the same residuals: the chunk-start
// states and e = v - u per token and state row in ckpt, the dq/dk/dg/dbeta partials per row block in the workspace
// and rec_reduce_kernel's fixed-order sums after them.
//
// One wave per state row, its 64 lanes striding the row's columns (lane l holds columns l, l + 64, ...): the row's
// state and its cotangent stay in LDS (Dk floats each), the step's k and q rows are read from global memory (the
// row block's waves read the same rows), and both dot products of a step are wave-wide sums in a fixed order
// (each lane's columns in order, then the lanes by DPP and lane swaps, every lane getting the same bits). The
// backward keeps the state at every 8th step of a chunk in the workspace (pass A) and re-forms each step's previous
// and current state from the nearest kept one (pass B), so neither the chunk's states nor a per-lane copy of the row
// has to fit anywhere. Per reverse step the block's waves hand their dq/dk column contributions to LDS and the block
// sums them over its rows in row order. The layout trades speed for reach: it is the fallback for widths no model
// of this family uses, not a tuned path.
#include <type_traits>

#include "gdn_common.h"
#include "gdn_kernels.h"

namespace qbgdn {
namespace {

constexpr int kSubW = 8;  // the backward keeps every kSubW-th state of a chunk

struct WideFwdArgs {
  FwdPtrs p;
  float* e_res;  // v - u per token and state row [tokens, Hv, Dv], after the states in ckpt (null without ckpt)
  int Hk, Hv, Dk, Dv, g_is_log, nblk, total;
  SeqTable tab;
};

struct WideBwdArgs {
  BwdPtrs p;
  const float* e_res;
  int Hk, Hv, Dk, Dv, g_is_log, nblk, total;
  float* dq_part;  // [BT, Hv, nblk, Dk]
  float* dk_part;
  float* dg_part;  // [BT, Hv, nblk]
  float* db_part;
  float* scratch;  // per block and row: kSubW kept states, then the previous and current state [kSubW + 2][Dk]
  SeqTable tab;
};

// Sum over the wave; every lane gets the same bits (each stage pairs lanes symmetrically).
__device__ __forceinline__ float wave_sum(float x) { return swap32_sum(swap16_sum(sum16(x))); }

// The decay factor and beta of a step.
template <typename InT>
__device__ __forceinline__ float2 step_scalars(const float* g, const InT* beta, int64_t i, int g_is_log) {
  const float gv = g[i];
  return float2{g_is_log ? expf(gv) : gv, IO<InT>::ld(beta, i)};
}

// Forward: rows per block R (one wave each). The row's state in LDS, R * Dk floats (dynamic).
template <typename InT, typename OutT, bool kKeepRows>
__global__ __launch_bounds__(256) void rec_wide_fwd_kernel(WideFwdArgs a) {
  extern __shared__ float wlds[];
  const int R = blockDim.x >> 6, Dk = a.Dk;
  const StateItem it = state_item(a.tab, blockIdx.x, a.nblk, a.Hv, a.Hk, a.total);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int row = it.blk * R + w;
  if (row >= a.Dv) return;  // no barriers here: a row past Dv has nothing to do
  const int hv = it.hv, hk = hv / (a.Hv / a.Hk);
  const Seq sq = seq_of(a.tab, it.n);
  const InT* q = static_cast<const InT*>(a.p.q);
  const InT* k = static_cast<const InT*>(a.p.k);
  const InT* v = static_cast<const InT*>(a.p.v);
  const InT* beta = static_cast<const InT*>(a.p.beta);
  OutT* y = static_cast<OutT*>(a.p.y);
  const int64_t SS = int64_t(a.Dv) * Dk;
  const int64_t srow = (int64_t(it.n) * a.Hv + hv) * SS + int64_t(row) * Dk;
  float* S = wlds + w * Dk;
  for (int c = lane; c < Dk; c += 64) S[c] = a.p.s0 ? a.p.s0[srow + c] : 0.f;

  const int nch = (sq.len + kChunk - 1) / kChunk;
  for (int ch = 0; ch < nch; ++ch) {
    const int t0 = ch * kChunk, L = min(kChunk, sq.len - t0);
    if (a.p.ckpt) {
      float* dst = a.p.ckpt + ((sq.slot0 + ch) * a.Hv + hv) * SS + int64_t(row) * Dk;
      for (int c = lane; c < Dk; c += 64) dst[c] = S[c];
    }
    for (int tt = 0; tt < L; ++tt) {
      const int64_t tok = sq.tok0 + t0 + tt, at = (tok * a.Hv + hv) * a.Dv + row;
      const InT* kr = k + (tok * a.Hk + hk) * Dk;
      const InT* qr = q + (tok * a.Hk + hk) * Dk;
      // Both dot products on the previous state, and k.q, as rec.hip forms them.
      float pa = 0.f, pb = 0.f, kq = 0.f;
      for (int c = lane; c < Dk; c += 64) {
        const float kc = IO<InT>::ld(kr, c), qc = IO<InT>::ld(qr, c), s = S[c];
        pa = fmaf(s, kc, pa), pb = fmaf(s, qc, pb), kq = fmaf(kc, qc, kq);
      }
      pa = wave_sum(pa), pb = wave_sum(pb), kq = wave_sum(kq);
      const float2 gb = step_scalars(a.p.g, beta, tok * a.Hv + hv, a.g_is_log);
      const float gt = gb.x, bt = gb.y;
      const float e = fmaf(-gt, pa, IO<InT>::ld(v, at));
      const float d = bt * e;
      const float yv = fmaf(gt, pb, d * kq);
      for (int c = lane; c < Dk; c += 64) S[c] = fmaf(gt, S[c], d * IO<InT>::ld(kr, c));
      if (lane == 0) {
        IO<OutT>::st(y, at, yv);
        if (a.e_res) a.e_res[at] = e;
      }
      if constexpr (kKeepRows) {  // the state after this token
        float* dst = a.p.rows + (tok * a.Hv + hv) * SS + int64_t(row) * Dk;
        for (int c = lane; c < Dk; c += 64) dst[c] = S[c];
      }
    }
  }
  if (a.p.s_out)
    for (int c = lane; c < Dk; c += 64) a.p.s_out[srow + c] = S[c];
}

// Backward: rows per block R (one wave each). LDS (dynamic): the rows' state cotangents [R][Dk], then each row's dq
// and dk column contributions of the current step [R][2 Dk], then per row dbeta and dg [R][2].
template <typename InT, typename OutT>
__global__ __launch_bounds__(256) void rec_wide_bwd_kernel(WideBwdArgs a) {
  extern __shared__ float wlds[];
  const int R = blockDim.x >> 6, Dk = a.Dk;
  const StateItem it = state_item(a.tab, blockIdx.x, a.nblk, a.Hv, a.Hk, a.total);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int row0 = it.blk * R, row = row0 + w, nlive = min(R, a.Dv - row0);
  const bool live = row < a.Dv;
  const int hv = it.hv, hk = hv / (a.Hv / a.Hk);
  const Seq sq = seq_of(a.tab, it.n);
  const InT* q = static_cast<const InT*>(a.p.q);
  const InT* k = static_cast<const InT*>(a.p.k);
  const OutT* dy = static_cast<const OutT*>(a.p.dy);
  const InT* beta = static_cast<const InT*>(a.p.beta);
  OutT* dv = static_cast<OutT*>(a.p.dv);
  const int64_t SS = int64_t(a.Dv) * Dk;
  const int64_t srow = (int64_t(it.n) * a.Hv + hv) * SS + int64_t(row) * Dk;
  float* dS = wlds + w * Dk;
  float* red = wlds + R * Dk;        // [R][2 Dk]
  float* rowv = red + 2 * R * Dk;    // [R][2]: dbeta, dg of the step
  // This row's workspace: the kept states, then the previous and current state of the step.
  float* keep = a.scratch + (int64_t(blockIdx.x) * R + w) * (kSubW + 2) * Dk;
  float* Sp = keep + kSubW * Dk;
  float* Sc = Sp + Dk;
  for (int c = lane; c < Dk; c += 64) dS[c] = (live && a.p.ds_out) ? a.p.ds_out[srow + c] : 0.f;

  // One step of the forward replay on a row held in global memory: x <- g x + beta e k (e the forward's v - u).
  auto advance = [&](float* x, int64_t tok) {
    const float2 gb = step_scalars(a.p.g, beta, tok * a.Hv + hv, a.g_is_log);
    const float d = gb.y * a.e_res[(tok * a.Hv + hv) * a.Dv + row];
    const InT* kr = k + (tok * a.Hk + hk) * Dk;
    for (int c = lane; c < Dk; c += 64) x[c] = gb.x * x[c] + d * IO<InT>::ld(kr, c);
  };

  const int nch = (sq.len + kChunk - 1) / kChunk;
  for (int ch = nch - 1; ch >= 0; --ch) {
    const int t0 = ch * kChunk, L = min(kChunk, sq.len - t0);
    const int64_t tokc = sq.tok0 + t0;
    // Pass A: the chunk's states from its checkpoint, every kSubW-th kept.
    if (live) {
      const float* src = a.p.ckpt + ((sq.slot0 + ch) * a.Hv + hv) * SS + int64_t(row) * Dk;
      for (int c = lane; c < Dk; c += 64) Sc[c] = src[c];
      for (int m = 0; m * kSubW < L; ++m) {
        float* km = keep + m * Dk;
        for (int c = lane; c < Dk; c += 64) km[c] = Sc[c];
        for (int j = 0; j < kSubW && m * kSubW + j < L; ++j) advance(Sc, tokc + m * kSubW + j);
      }
    }
    // Pass B: the reverse steps (reference :97-141), each step's previous state re-formed from the nearest kept one.
    for (int tt = L - 1; tt >= 0; --tt) {
      const int64_t tok = tokc + tt;
      float dd = 0.f, dg = 0.f, bt = 0.f, e = 0.f;
      if (live) {
        const int m = tt / kSubW;
        const float* km = keep + m * Dk;
        for (int c = lane; c < Dk; c += 64) Sp[c] = km[c];
        for (int j = m * kSubW; j < tt; ++j) advance(Sp, tokc + j);
        const float2 gb = step_scalars(a.p.g, beta, tok * a.Hv + hv, a.g_is_log);
        const float gt = gb.x;
        bt = gb.y;
        const int64_t at = (tok * a.Hv + hv) * a.Dv + row;
        e = a.e_res[at];
        const float d = bt * e, dyt = IO<OutT>::ld(dy, at);
        const InT* kr = k + (tok * a.Hk + hk) * Dk;
        const InT* qr = q + (tok * a.Hk + hk) * Dk;
        float* rq = red + w * 2 * Dk;
        // dS += dy q^T; the dq contribution dy S (S the state after the step); dd = dS k.
        for (int c = lane; c < Dk; c += 64) {
          const float kc = IO<InT>::ld(kr, c);
          Sc[c] = gt * Sp[c] + d * kc;
          dS[c] += dyt * IO<InT>::ld(qr, c);
          rq[c] = dyt * Sc[c];
          dd += dS[c] * kc;
        }
        dd = wave_sum(dd);
        const float du = -bt * dd, dug = du * gt;
        // The dk contribution dS d + du g S_prev; dS of the decayed state; dg = sum dS~ * S_prev; dS of S_prev.
        for (int c = lane; c < Dk; c += 64) {
          const float kc = IO<InT>::ld(kr, c);
          rq[Dk + c] = dS[c] * d + dug * Sp[c];
          dS[c] += du * kc;
          dg += dS[c] * Sp[c];
          dS[c] *= gt;
        }
        dg = wave_sum(dg);
        if (lane == 0) {
          IO<OutT>::st(dv, at, bt * dd);
          rowv[2 * w] = dd * e, rowv[2 * w + 1] = dg;
        }
      }
      __syncthreads();
      // The block's sums over its rows, in row order.
      const int64_t pr = (tok * a.Hv + hv) * a.nblk + it.blk;
      for (int col = tid; col < 2 * Dk; col += blockDim.x) {
        float acc = 0.f;
        for (int r = 0; r < nlive; ++r) acc += red[r * 2 * Dk + col];
        (col < Dk ? a.dq_part + pr * Dk + col : a.dk_part + pr * Dk + col - Dk)[0] = acc;
      }
      if (tid < 2) {
        float acc = 0.f;
        for (int r = 0; r < nlive; ++r) acc += rowv[2 * r + tid];
        (tid == 0 ? a.db_part : a.dg_part)[pr] = acc;
      }
      __syncthreads();
    }
  }
  if (live && a.p.ds0)
    for (int c = lane; c < Dk; c += 64) a.p.ds0[srow + c] = dS[c];
}

}  // namespace

int rec_wide_fwd_rows(int Dk) { return Dk <= 2048 ? 4 : 2; }
int rec_wide_bwd_rows(int Dk) { return Dk <= 1024 ? 4 : Dk <= 2048 ? 2 : 1; }

size_t rec_wide_scratch_bytes(const Problem& p) {
  const int R = rec_wide_bwd_rows(p.Dk);
  const size_t blocks = size_t((p.Dv + R - 1) / R) * p.Hv * p.N;
  return blocks * R * (kSubW + 2) * size_t(p.Dk) * sizeof(float);
}

template <typename InT, typename OutT>
hipError_t rec_wide_fwd(const Problem& p, const FwdPtrs& ptrs, hipStream_t s) {
  WideFwdArgs a;
  a.p = ptrs;
  a.e_res = ptrs.ckpt ? ptrs.ckpt + int64_t(p.NC) * p.Hv * p.Dv * p.Dk : nullptr;
  a.Hk = p.Hk, a.Hv = p.Hv, a.Dk = p.Dk, a.Dv = p.Dv, a.g_is_log = p.g_is_log;
  const int R = rec_wide_fwd_rows(p.Dk);
  a.nblk = (p.Dv + R - 1) / R;
  a.total = a.nblk * p.Hv * p.N;
  a.tab = p.tab;
  if (a.total == 0) return hipSuccess;
  const size_t lds = size_t(R) * p.Dk * sizeof(float);
  if (ptrs.rows)
    hipLaunchKernelGGL((rec_wide_fwd_kernel<InT, OutT, true>), dim3(a.total), dim3(64 * R), lds, s, a);
  else
    hipLaunchKernelGGL((rec_wide_fwd_kernel<InT, OutT, false>), dim3(a.total), dim3(64 * R), lds, s, a);
  return hipGetLastError();
}

template <typename InT, typename OutT>
hipError_t rec_wide_bwd(const Problem& p, const BwdPtrs& ptrs, float* dq_part, float* dk_part, float* dg_part,
                        float* db_part, float* scratch, int nblk, hipStream_t s) {
  WideBwdArgs a;
  a.p = ptrs;
  a.e_res = ptrs.ckpt + int64_t(p.NC) * p.Hv * p.Dv * p.Dk;
  a.Hk = p.Hk, a.Hv = p.Hv, a.Dk = p.Dk, a.Dv = p.Dv, a.g_is_log = p.g_is_log;
  a.nblk = nblk;
  a.total = nblk * p.Hv * p.N;
  a.dq_part = dq_part, a.dk_part = dk_part, a.dg_part = dg_part, a.db_part = db_part;
  a.scratch = scratch;
  a.tab = p.tab;
  if (a.total == 0) return hipSuccess;
  const int R = rec_wide_bwd_rows(p.Dk);
  const size_t lds = (size_t(R) * 3 * p.Dk + 2 * R) * sizeof(float);
  hipLaunchKernelGGL((rec_wide_bwd_kernel<InT, OutT>), dim3(a.total), dim3(64 * R), lds, s, a);
  return hipGetLastError();
}

template hipError_t rec_wide_fwd<float, float>(const Problem&, const FwdPtrs&, hipStream_t);
template hipError_t rec_wide_fwd<bf16_t, bf16_t>(const Problem&, const FwdPtrs&, hipStream_t);
template hipError_t rec_wide_fwd<bf16_t, float>(const Problem&, const FwdPtrs&, hipStream_t);
template hipError_t rec_wide_bwd<float, float>(const Problem&, const BwdPtrs&, float*, float*, float*, float*, float*,
                                               int, hipStream_t);
template hipError_t rec_wide_bwd<bf16_t, bf16_t>(const Problem&, const BwdPtrs&, float*, float*, float*, float*,
                                                 float*, int, hipStream_t);
template hipError_t rec_wide_bwd<bf16_t, float>(const Problem&, const BwdPtrs&, float*, float*, float*, float*,
                                                float*, int, hipStream_t);

}  // namespace qbgdn
