// Chunked design, kernel 5 (only when g is given as the decay factor): dL/dg where the factor is tiny or zero.
//
// The gradient kernel forms dL/dG_t, the gradient of the log-decay, as a reverse cumulative sum of terms of both
// signs, and divides it by g_t. Where g_t is tiny the quotient magnifies the sum's rounding without bound, and at
// g_t = 0 it is 0/0. The gradient itself is finite there: the loss is affine in each g_t, and
//   dL/dg_t = <M_t, S_{t-1}>   (summed over the state's rows and columns)
// with S_{t-1} the state before step t and M_t the cotangent of the decayed state g_t S_{t-1}, the quantity the
// reference's backward sweep forms step by step (src/delta_grad.cpp:104-119). For each (chunk slot, value head)
// whose chunk holds a factor below kTiny, this kernel replays the chunk's rows: forward from the checkpoint to the
// flagged steps (keeping S_{t-1} there), then back from the chunk-end cotangent the backward state pass stored,
// forming M_t and the inner product at each flagged step. Rows are independent, so 16 lanes hold a row (8 columns
// each) and a wave four rows; sums over the 16 lanes of a row are DPP reductions. Float32 throughout, fixed
// summation order. Chunks without a tiny factor return after reading their 64 factors.
#include <type_traits>

#include "chunk_common.h"
#include "chunk_kernels.h"

namespace qbgdn {
namespace {

constexpr int kThreads = 512;        // 8 waves x 4 rows: 32 state rows per pass
constexpr int kRows = 32;
constexpr int kBatch = 4;            // flagged steps per forward/backward replay
constexpr float kTiny = 0x1p-10f;    // factors below this take this kernel's value

template <typename OutT>
__global__ __launch_bounds__(kThreads) void chunk_dgfix_kernel(ChunkArgs a) {
  constexpr int Dk = 128;
  __shared__ float Ks[kC][Dk], Qs[kC][Dk];      // k and q rows of the chunk (zeros past its end)
  __shared__ float Vs[kC][kRows], Ys[kC][kRows];  // v and dy of the pass's state rows
  __shared__ float Gs[kC], Bs[kC];
  __shared__ int fl[kC];                          // flagged steps, ascending
  __shared__ int nfl;
  __shared__ float xs[kThreads / 64][4][kBatch];  // per wave and row group: the rows' sums so far

  const int total = int(a.lay.NC) * a.Hv;
  const int64_t slot = blockIdx.x / a.Hv;
  const int hv = blockIdx.x % a.Hv, hk = hv / (a.Hv / a.Hk);
  if (blockIdx.x >= total) return;
  const SlotPos sp = slot_pos(a.tab, slot);
  const int L = sp.L;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int sk = a.Hk * Dk, sv = a.Hv * a.Dv;

  if (tid < kC) {  // wave 0: the factors, beta and the flagged steps
    const int t = tid;
    const float gx = t < L ? a.g[(sp.tok + t) * a.Hv + hv] : 1.f;
    Gs[t] = gx;
    Bs[t] = t < L ? bf16_to_f32(a.beta[(sp.tok + t) * a.Hv + hv]) : 0.f;
    const bool f = t < L && !(gx >= kTiny);
    const uint64_t m = __ballot(f);
    if (f) fl[__popcll(m & ((uint64_t(1) << t) - 1))] = t;
    if (t == 0) nfl = __popcll(m);
  }
  __syncthreads();
  const int nf = nfl;
  if (nf == 0) return;

  for (int e = tid; e < kC * Dk; e += kThreads) {
    const int t = e / Dk, c = e % Dk;
    const int64_t at = (sp.tok + t) * sk + hk * Dk + c;
    Ks[t][c] = t < L ? bf16_to_f32(a.k[at]) : 0.f;
    Qs[t][c] = t < L ? bf16_to_f32(a.q[at]) : 0.f;
  }
  const OutT* dy = static_cast<const OutT*>(a.dy);
  const int rl = 4 * w + (lane >> 4), c0 = 8 * (lane & 15);
  const float* S0 = a.ckpt + (slot * a.Hv + hv) * int64_t(a.Dv) * Dk;
  const float* dSe = a.dsend + (slot * a.Hv + hv) * int64_t(a.Dv) * Dk;

  for (int f0 = 0; f0 < nf; f0 += kBatch) {
    const int nb = min(kBatch, nf - f0);
    float xr[kBatch] = {0.f, 0.f, 0.f, 0.f};  // this row group's sum over its rows so far
    for (int r0 = 0; r0 < a.Dv; r0 += kRows) {
      __syncthreads();  // the previous pass is done with Vs, Ys
      for (int e = tid; e < kC * kRows; e += kThreads) {
        const int t = e / kRows, r = e % kRows;
        const int64_t at = (sp.tok + t) * sv + hv * a.Dv + r0 + r;
        Vs[t][r] = t < L ? bf16_to_f32(a.v[at]) : 0.f;
        Ys[t][r] = t < L ? IO<OutT>::ld(dy, at) : 0.f;
      }
      __syncthreads();
      const int r = r0 + rl;
      // Forward: s = S_{t-1} row r, this lane's 8 columns; kept at each flagged step of the batch.
      float s[8], sv8[kBatch][8];
#pragma unroll
      for (int j = 0; j < 8; ++j) s[j] = S0[int64_t(r) * Dk + c0 + j];
      int fi = 0;
      const int tend = fl[f0 + nb - 1];
      for (int t = 0; t < tend; ++t) {
        if (t == fl[f0 + fi]) {
#pragma unroll
          for (int b = 0; b < kBatch; ++b)
            if (b == fi)
#pragma unroll
              for (int j = 0; j < 8; ++j) sv8[b][j] = s[j];
          ++fi;
        }
        const float gt = Gs[t];
        float u = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          s[j] *= gt;
          u += s[j] * Ks[t][c0 + j];
        }
        u = sum16(u);
        const float d = Bs[t] * (Vs[t][rl] - u);
#pragma unroll
        for (int j = 0; j < 8; ++j) s[j] += d * Ks[t][c0 + j];
      }
#pragma unroll
      for (int b = 0; b < kBatch; ++b)  // the last flagged step of the batch ends the loop
        if (b == nb - 1)
#pragma unroll
          for (int j = 0; j < 8; ++j) sv8[b][j] = s[j];
      // Backward from the chunk end: m = cotangent of S_t row r (its y term added), then of the decayed state.
      float m[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) m[j] = dSe[int64_t(r) * Dk + c0 + j];
      fi = nb - 1;
      for (int t = L - 1; t >= fl[f0]; --t) {
        const float yt = Ys[t][rl];
        float u = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          m[j] += yt * Qs[t][c0 + j];
          u += m[j] * Ks[t][c0 + j];
        }
        u = Bs[t] * sum16(u);
#pragma unroll
        for (int j = 0; j < 8; ++j) m[j] -= u * Ks[t][c0 + j];  // M_t
        if (t == fl[f0 + fi]) {
          float x = 0.f;
#pragma unroll
          for (int b = 0; b < kBatch; ++b)
            if (b == fi)
#pragma unroll
              for (int j = 0; j < 8; ++j) x += m[j] * sv8[b][j];
          x = sum16(x);
#pragma unroll
          for (int b = 0; b < kBatch; ++b)
            if (b == fi) xr[b] += x;
          --fi;
        }
        const float gt = Gs[t];
#pragma unroll
        for (int j = 0; j < 8; ++j) m[j] *= gt;
      }
    }
    if ((lane & 15) == 0) {
#pragma unroll
      for (int b = 0; b < kBatch; ++b) xs[w][lane >> 4][b] = xr[b];
    }
    __syncthreads();
    if (tid < nb) {  // the sum over every row, in a fixed order
      float x = 0.f;
      for (int ww = 0; ww < kThreads / 64; ++ww)
        for (int q = 0; q < 4; ++q) x += xs[ww][q][tid];
      a.dg[(sp.tok + fl[f0 + tid]) * a.Hv + hv] = x;
    }
  }
}

}  // namespace

hipError_t launch_chunk_dgfix(const ChunkArgs& a, bool out_bf16, hipStream_t s) {
  const int total = int(a.lay.NC) * a.Hv;
  if (total == 0) return hipSuccess;
  if (out_bf16)
    hipLaunchKernelGGL(chunk_dgfix_kernel<bf16_t>, dim3(total), dim3(kThreads), 0, s, a);
  else
    hipLaunchKernelGGL(chunk_dgfix_kernel<float>, dim3(total), dim3(kThreads), 0, s, a);
  return hipGetLastError();
}

}  // namespace qbgdn
