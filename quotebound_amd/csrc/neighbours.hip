// The layer's pointwise neighbours of the recurrence, each one pass over its rows (reference src/deltanet.cpp):
//   prologue  q = s_q * rms_norm(q_raw), k = s_k * rms_norm(k_raw)   (:94-97: s_q = 1/Dk and s_k = Dk^-1/2 in the
//             activation dtype, rms_norm without weight and eps 1e-6), beta = sigmoid(b) (:99), and
//             log_decay = -exp(A_log) * softplus(a + dt_bias)          (:22-33, :100: compute_g, whose final exp the
//             recurrence takes itself when fed the log-decay)
//   epilogue  o = silu(z) * rms_norm(y, w, eps)                       (:35-45, :122: the gated RMSNorm)
// and their backward. With bf16 activations the forward rounds where the reference's ops do, each op's output
// taking the activation dtype: rms_norm's output, then its product with the scale; a + dt_bias, then its softplus;
// the rms_norm's normalised row, then its product with the weight, then that with silu(z). Arithmetic inside an op is float32. The backward is float32
// throughout, with one rounding of each output; the parameter gradients (A_log, dt_bias per value head, w per
// column) are summed over tokens in a fixed order: per-block partials, then one pass over the blocks in order.
//
// One wave per row of D = 64 E elements (E = 1, 2, 4): lane l holds elements E l .. E l + E - 1, so a row is one
// contiguous read; the sum of squares is a fixed-order reduction over the wave.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "gdn_common.h"
#include "neighbours.h"

namespace qbgdn {
namespace {

constexpr float kNormEps = 1e-6f;  // the q/k rms_norm's eps (src/deltanet.cpp:96-97)

template <typename T>
__device__ __forceinline__ float rnd(float x) {  // the activation dtype's rounding
  if constexpr (sizeof(T) == 2) return bf16_to_f32(f32_to_bf16(x));
  return x;
}

__device__ __forceinline__ float wave_sum(float x) {
  x = sum16(x);
  x += __shfl_xor(x, 16);
  x += __shfl_xor(x, 32);
  return x;
}

__device__ __forceinline__ float sigmoidf(float x) { return 1.f / (1.f + expf(-x)); }
__device__ __forceinline__ float softplusf(float x) { return fmaxf(x, 0.f) + log1pf(expf(-fabsf(x))); }

template <typename T, int E>
__device__ __forceinline__ void load_row(const T* p, float (&x)[E]) {
#pragma unroll
  for (int e = 0; e < E; ++e) x[e] = IO<T>::ld(p, e);
}

// Rows of q_raw then k_raw (2 R rows of D): out = rnd(scale * rnd(x * rho)), rho = (mean(x^2) + eps)^-1/2.
template <typename T, int E>
__global__ __launch_bounds__(256) void qk_norm_fwd(const T* __restrict__ qr, const T* __restrict__ kr,
                                                   T* __restrict__ q, T* __restrict__ k, int64_t R, float sq,
                                                   float sk) {
  constexpr int D = 64 * E;
  const int lane = threadIdx.x & 63;
  const int64_t row = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= 2 * R) return;
  const bool isk = row >= R;
  const int64_t r = isk ? row - R : row;
  const T* src = (isk ? kr : qr) + r * D + E * lane;
  T* dst = (isk ? k : q) + r * D + E * lane;
  const float s = isk ? sk : sq;
  float x[E];
  load_row<T, E>(src, x);
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) ss += x[e] * x[e];
  const float rho = 1.f / sqrtf(wave_sum(ss) / D + kNormEps);
#pragma unroll
  for (int e = 0; e < E; ++e) IO<T>::st(dst, e, rnd<T>(s * rnd<T>(x[e] * rho)));
}

// beta and the log-decay per (token, value head).
template <typename T>
__global__ __launch_bounds__(256) void gates_fwd(const T* __restrict__ a, const T* __restrict__ b,
                                                 const float* __restrict__ a_log, const float* __restrict__ dt_bias,
                                                 T* __restrict__ beta, float* __restrict__ log_decay, int64_t n,
                                                 int Hv) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  const int h = int(i % Hv);
  IO<T>::st(beta, i, sigmoidf(IO<T>::ld(b, i)));
  const float x = rnd<T>(IO<T>::ld(a, i) + dt_bias[h]);
  log_decay[i] = -expf(a_log[h]) * rnd<T>(softplusf(x));
}

// The backward of qk_norm_fwd: g = scale * dout, dx = rho g - rho^3 x (sum g x) / D.
template <typename T, int E>
__global__ __launch_bounds__(256) void qk_norm_bwd(const T* __restrict__ qr, const T* __restrict__ kr,
                                                   const T* __restrict__ dq, const T* __restrict__ dk,
                                                   T* __restrict__ dqr, T* __restrict__ dkr, int64_t R, float sq,
                                                   float sk) {
  constexpr int D = 64 * E;
  const int lane = threadIdx.x & 63;
  const int64_t row = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= 2 * R) return;
  const bool isk = row >= R;
  const int64_t r = isk ? row - R : row;
  const int64_t off = r * D + E * lane;
  const float s = isk ? sk : sq;
  float x[E], gd[E];
  load_row<T, E>((isk ? kr : qr) + off, x);
  load_row<T, E>((isk ? dk : dq) + off, gd);
  float ss = 0.f, gx = 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    gd[e] *= s;
    ss += x[e] * x[e];
    gx += gd[e] * x[e];
  }
  const float rho = 1.f / sqrtf(wave_sum(ss) / D + kNormEps);
  const float c = rho * rho * rho * wave_sum(gx) / D;
  T* out = (isk ? dkr : dqr) + off;
#pragma unroll
  for (int e = 0; e < E; ++e) IO<T>::st(out, e, rho * gd[e] - c * x[e]);
}

// The backward of gates_fwd for 64 consecutive tokens of one value head (one wave): db, da, and the tile's partial
// sums of dA_log = sum dlog_decay * log_decay and ddt_bias = sum da.
template <typename T>
__global__ __launch_bounds__(64) void gates_bwd(const T* __restrict__ a, const T* __restrict__ b,
                                                const float* __restrict__ a_log, const float* __restrict__ dt_bias,
                                                const T* __restrict__ dbeta, const float* __restrict__ dld,
                                                T* __restrict__ da, T* __restrict__ db, float* __restrict__ part,
                                                int64_t BT, int Hv) {
  const int h = blockIdx.y;
  const int64_t t = int64_t(blockIdx.x) * 64 + threadIdx.x;
  float pa = 0.f, pd = 0.f;
  if (t < BT) {
    const int64_t i = t * Hv + h;
    const float sb = sigmoidf(IO<T>::ld(b, i));
    IO<T>::st(db, i, IO<T>::ld(dbeta, i) * sb * (1.f - sb));
    const float ea = expf(a_log[h]);
    const float x = rnd<T>(IO<T>::ld(a, i) + dt_bias[h]);
    const float g = dld[i];
    const float dx = -g * ea * sigmoidf(x);
    IO<T>::st(da, i, dx);
    pa = g * (-ea * rnd<T>(softplusf(x)));  // d log_decay / d A_log = log_decay
    pd = dx;
  }
  pa = wave_sum(pa), pd = wave_sum(pd);
  if (threadIdx.x == 0) {
    part[(int64_t(blockIdx.x) * Hv + h) * 2] = pa;
    part[(int64_t(blockIdx.x) * Hv + h) * 2 + 1] = pd;
  }
}

// out[c] = sum over parts p of part[p * stride + c * step + comp], for c < width, in a fixed order: 64 columns per
// block, wave v summing the parts p = v mod 4 in increasing order, then the four waves' sums in order.
__global__ __launch_bounds__(256) void sum_parts(const float* __restrict__ part, int64_t nparts, int stride,
                                                 int step, int comp, int width, float* __restrict__ out) {
  __shared__ float red[4][64];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int c = blockIdx.x * 64 + lane;
  float s = 0.f;
  if (c < width)
    for (int64_t p = wv; p < nparts; p += 4) s += part[p * stride + int64_t(c) * step + comp];
  red[wv][lane] = s;
  __syncthreads();
  if (wv == 0 && c < width) out[c] = ((red[0][lane] + red[1][lane]) + red[2][lane]) + red[3][lane];
}

// The gated RMSNorm: o = rnd(silu(z) * rnd(w * rnd(y * rho))), one row of Dv per wave (rms_norm normalises, takes
// the output dtype, then multiplies by its weight).
template <typename T, int E>
__global__ __launch_bounds__(256) void gated_norm_fwd(const T* __restrict__ y, const T* __restrict__ z,
                                                      const float* __restrict__ w, float eps, T* __restrict__ o,
                                                      int64_t R) {
  constexpr int D = 64 * E;
  const int lane = threadIdx.x & 63;
  const int64_t row = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= R) return;
  const int64_t off = row * D + E * lane;
  float x[E], zz[E];
  load_row<T, E>(y + off, x);
  load_row<T, E>(z + off, zz);
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < E; ++e) ss += x[e] * x[e];
  const float rho = 1.f / sqrtf(wave_sum(ss) / D + eps);
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const float n = rnd<T>(w[E * lane + e] * rnd<T>(x[e] * rho));
    IO<T>::st(o + off, e, rnd<T>(zz[e] * sigmoidf(zz[e]) * n));
  }
}

// Its backward over groups of 64 rows (16 per wave), block b taking groups b, b + gridDim.x, ...: dz = do n silu'(z),
// dy through the norm, and the block's partial dw per column (summed over its rows in a fixed order: each wave over
// its rows, then the four waves in order).
template <typename T, int E>
__global__ __launch_bounds__(256) void gated_norm_bwd(const T* __restrict__ y, const T* __restrict__ z,
                                                      const float* __restrict__ w, float eps,
                                                      const T* __restrict__ dout, T* __restrict__ dy,
                                                      T* __restrict__ dz, float* __restrict__ part, int64_t R) {
  constexpr int D = 64 * E;
  __shared__ float acc[4][D];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  float pw[E];
  float wl[E];
#pragma unroll
  for (int e = 0; e < E; ++e) pw[e] = 0.f, wl[e] = w[E * lane + e];
  for (int64_t grp = blockIdx.x; grp * 64 < R; grp += gridDim.x) {
    for (int k = 0; k < 16; ++k) {
      const int64_t row = grp * 64 + wv * 16 + k;
      if (row >= R) break;
      const int64_t off = row * D + E * lane;
      float x[E], zz[E], go[E];
      load_row<T, E>(y + off, x);
      load_row<T, E>(z + off, zz);
      load_row<T, E>(dout + off, go);
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < E; ++e) ss += x[e] * x[e];
      const float rho = 1.f / sqrtf(wave_sum(ss) / D + eps);
      float g[E], gx = 0.f;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const float sg = sigmoidf(zz[e]), silu = zz[e] * sg, nh = x[e] * rho;
        IO<T>::st(dz + off, e, go[e] * nh * wl[e] * sg * (1.f + zz[e] * (1.f - sg)));
        const float dn = go[e] * silu;
        pw[e] += dn * nh;
        g[e] = dn * wl[e];
        gx += g[e] * x[e];
      }
      const float c = rho * rho * rho * wave_sum(gx) / D;
#pragma unroll
      for (int e = 0; e < E; ++e) IO<T>::st(dy + off, e, rho * g[e] - c * x[e]);
    }
  }
#pragma unroll
  for (int e = 0; e < E; ++e) acc[wv][E * lane + e] = pw[e];
  __syncthreads();
  for (int c = threadIdx.x; c < D; c += 256)
    part[int64_t(blockIdx.x) * D + c] = ((acc[0][c] + acc[1][c]) + acc[2][c]) + acc[3][c];
}

}  // namespace

// Host side -------------------------------------------------------------------------------------------------------

namespace {

// Blocks of the gated-norm backward: one per 64 rows up to 1024 (four per CU), so the partial dw stays small.
int64_t norm_bwd_blocks(int64_t R) {
  const int64_t groups = (R + 63) / 64;
  return groups < 1024 ? groups : 1024;
}

template <int E, typename T>
hipError_t qk_fwd_e(const NbProblem& p, const NbPrologue& x, hipStream_t s) {
  const int64_t R = p.BT * p.Hk;
  const unsigned blocks = unsigned((2 * R + 3) / 4);
  if (blocks)
    hipLaunchKernelGGL((qk_norm_fwd<T, E>), dim3(blocks), dim3(256), 0, s, static_cast<const T*>(x.q_raw),
                       static_cast<const T*>(x.k_raw), static_cast<T*>(x.q), static_cast<T*>(x.k), R, p.scale_q,
                       p.scale_k);
  return hipGetLastError();
}

template <int E, typename T>
hipError_t qk_bwd_e(const NbProblem& p, const NbPrologueGrad& x, hipStream_t s) {
  const int64_t R = p.BT * p.Hk;
  const unsigned blocks = unsigned((2 * R + 3) / 4);
  if (blocks)
    hipLaunchKernelGGL((qk_norm_bwd<T, E>), dim3(blocks), dim3(256), 0, s, static_cast<const T*>(x.q_raw),
                       static_cast<const T*>(x.k_raw), static_cast<const T*>(x.dq), static_cast<const T*>(x.dk),
                       static_cast<T*>(x.dq_raw), static_cast<T*>(x.dk_raw), R, p.scale_q, p.scale_k);
  return hipGetLastError();
}

template <int E, typename T>
hipError_t gn_fwd_e(const NbProblem& p, const NbEpilogue& x, hipStream_t s) {
  const int64_t R = p.BT * p.Hv;
  const unsigned blocks = unsigned((R + 3) / 4);
  if (blocks)
    hipLaunchKernelGGL((gated_norm_fwd<T, E>), dim3(blocks), dim3(256), 0, s, static_cast<const T*>(x.y),
                       static_cast<const T*>(x.z), x.w, x.eps, static_cast<T*>(x.o), R);
  return hipGetLastError();
}

template <int E, typename T>
hipError_t gn_bwd_e(const NbProblem& p, const NbEpilogueGrad& x, void* ws, hipStream_t s) {
  const int64_t R = p.BT * p.Hv;
  const int64_t blocks = norm_bwd_blocks(R);
  float* part = static_cast<float*>(ws);
  if (blocks) {
    hipLaunchKernelGGL((gated_norm_bwd<T, E>), dim3(unsigned(blocks)), dim3(256), 0, s, static_cast<const T*>(x.y),
                       static_cast<const T*>(x.z), x.w, x.eps, static_cast<const T*>(x.dout), static_cast<T*>(x.dy),
                       static_cast<T*>(x.dz), part, R);
    hipLaunchKernelGGL(sum_parts, dim3(unsigned((p.Dv + 63) / 64)), dim3(256), 0, s, part, blocks, p.Dv, 1, 0,
                       p.Dv, x.dw);
  } else {  // no rows: zeros (a sum over no parts)
    hipLaunchKernelGGL(sum_parts, dim3(unsigned((p.Dv + 63) / 64)), dim3(256), 0, s, part, 0, p.Dv, 1, 0, p.Dv,
                       x.dw);
  }
  return hipGetLastError();
}

template <typename F>
hipError_t by_width(int D, F&& f) {
  switch (D) {
    case 64: return f(std::integral_constant<int, 1>{});
    case 128: return f(std::integral_constant<int, 2>{});
    case 256: return f(std::integral_constant<int, 4>{});
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

const char* nb_supports(const NbProblem& p) {
  if (p.Dk != 64 && p.Dk != 128 && p.Dk != 256) return "the neighbour kernels need Dk of 64, 128 or 256";
  if (p.Dv != 64 && p.Dv != 128 && p.Dv != 256) return "the neighbour kernels need Dv of 64, 128 or 256";
  return nullptr;
}

size_t nb_workspace_bytes(const NbProblem& p) {
  const size_t gates = size_t((p.BT + 63) / 64) * p.Hv * 2 * 4;
  const size_t norm = size_t(norm_bwd_blocks(p.BT * p.Hv)) * p.Dv * 4;
  return gates > norm ? gates : norm;
}

hipError_t nb_prologue_fwd(const NbProblem& p, const NbPrologue& x, hipStream_t s) {
  hipError_t e = by_width(p.Dk, [&](auto ec) {
    return p.bf16 ? qk_fwd_e<decltype(ec)::value, bf16_t>(p, x, s) : qk_fwd_e<decltype(ec)::value, float>(p, x, s);
  });
  if (e != hipSuccess) return e;
  const int64_t n = p.BT * p.Hv;
  if (n) {
    const dim3 grid(unsigned((n + 255) / 256));
    if (p.bf16)
      hipLaunchKernelGGL(gates_fwd<bf16_t>, grid, dim3(256), 0, s, static_cast<const bf16_t*>(x.a),
                         static_cast<const bf16_t*>(x.b), x.a_log, x.dt_bias, static_cast<bf16_t*>(x.beta),
                         x.log_decay, n, p.Hv);
    else
      hipLaunchKernelGGL(gates_fwd<float>, grid, dim3(256), 0, s, static_cast<const float*>(x.a),
                         static_cast<const float*>(x.b), x.a_log, x.dt_bias, static_cast<float*>(x.beta),
                         x.log_decay, n, p.Hv);
  }
  return hipGetLastError();
}

hipError_t nb_prologue_bwd(const NbProblem& p, const NbPrologueGrad& x, void* ws, hipStream_t s) {
  hipError_t e = by_width(p.Dk, [&](auto ec) {
    return p.bf16 ? qk_bwd_e<decltype(ec)::value, bf16_t>(p, x, s) : qk_bwd_e<decltype(ec)::value, float>(p, x, s);
  });
  if (e != hipSuccess) return e;
  const int64_t tiles = (p.BT + 63) / 64;
  float* part = static_cast<float*>(ws);
  const dim3 g2(unsigned((p.Hv + 63) / 64));
  if (tiles) {
    const dim3 grid(unsigned(tiles), unsigned(p.Hv));
    if (p.bf16)
      hipLaunchKernelGGL(gates_bwd<bf16_t>, grid, dim3(64), 0, s, static_cast<const bf16_t*>(x.a),
                         static_cast<const bf16_t*>(x.b), x.a_log, x.dt_bias, static_cast<const bf16_t*>(x.dbeta),
                         x.dlog_decay, static_cast<bf16_t*>(x.da), static_cast<bf16_t*>(x.db), part, p.BT, p.Hv);
    else
      hipLaunchKernelGGL(gates_bwd<float>, grid, dim3(64), 0, s, static_cast<const float*>(x.a),
                         static_cast<const float*>(x.b), x.a_log, x.dt_bias, static_cast<const float*>(x.dbeta),
                         x.dlog_decay, static_cast<float*>(x.da), static_cast<float*>(x.db), part, p.BT, p.Hv);
  }
  // (With no tokens, sums over no parts: zeros.)
  hipLaunchKernelGGL(sum_parts, g2, dim3(256), 0, s, part, tiles, p.Hv * 2, 2, 0, p.Hv, x.da_log);
  hipLaunchKernelGGL(sum_parts, g2, dim3(256), 0, s, part, tiles, p.Hv * 2, 2, 1, p.Hv, x.ddt_bias);
  return hipGetLastError();
}

hipError_t nb_epilogue_fwd(const NbProblem& p, const NbEpilogue& x, hipStream_t s) {
  return by_width(p.Dv, [&](auto ec) {
    return p.bf16 ? gn_fwd_e<decltype(ec)::value, bf16_t>(p, x, s) : gn_fwd_e<decltype(ec)::value, float>(p, x, s);
  });
}

hipError_t nb_epilogue_bwd(const NbProblem& p, const NbEpilogueGrad& x, void* ws, hipStream_t s) {
  return by_width(p.Dv, [&](auto ec) {
    return p.bf16 ? gn_bwd_e<decltype(ec)::value, bf16_t>(p, x, ws, s)
                  : gn_bwd_e<decltype(ec)::value, float>(p, x, ws, s);
  });
}

}  // namespace qbgdn
