// The layer's pointwise neighbours of the recurrence, each one pass over its rows (reference src/deltanet.cpp):
//   prologue  q = s_q * rms_norm(q_raw), k = s_k * rms_norm(k_raw)   (:94-97: s_q = 1/Dk and s_k = Dk^-1/2 in the
//             activation dtype, rms_norm without weight and eps 1e-6), beta = sigmoid(b) (:99), and
//             log_decay = -exp(A_log) * softplus(a + dt_bias)          (:22-33, :100: compute_g, whose final exp the
//             recurrence takes itself when fed the log-decay)
//   epilogue  o = silu(z) * rms_norm(y, w, eps)                       (:35-45, :122: the gated RMSNorm)
// and their backward. With bf16 activations the forward rounds where the reference's ops do, each op's output
// taking its inputs' dtype: rms_norm's normalised row, then its product with the scale; a + dt_bias, then its
// softplus; and o once (the gated rms_norm's weight is float32, so its output is float32 until the product with
// silu(z) takes the activation dtype). Arithmetic inside an op is float32. The backward is float32 throughout, with
// one rounding of each output; the parameter gradients (A_log, dt_bias per value head, w per column) are summed over
// tokens in a fixed order: per-block partials, then one pass over the blocks in order.
//
// Rows of D = 64, 128 or 256 elements: a lane holds 8 consecutive elements (one 16-byte load in bf16), a row takes
// D / 8 consecutive lanes and a group of 64 / (D / 8) rows fills a wave; a wave of the one-pass kernels takes two
// such groups, issuing both groups' loads before it computes. The sum of squares is a fixed-order reduction over the
// row's lanes. Lanes past the last row compute on a copy of the last row and store nothing, so every lane takes part in
// the reductions.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "gdn_common.h"
#include "neighbours.h"
#include "prologue_math.h"

namespace qbgdn {
namespace {

constexpr int kVec = 8;            // elements per lane
constexpr int kNormBwdBlocks = 256;  // gated-norm backward: at most one block of 16 waves per CU
constexpr int kGateSteps = 4;      // gates backward: steps per thread, so a tile is 4 (256 / Hv) tokens
constexpr int kSlots = 2;          // row groups per wave in the one-pass kernels, their loads issued together

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Round to nearest even bf16 in hardware (v_cvt_pk_bf16_f32), two values per instruction.
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}

// Sum over aligned groups of L consecutive lanes (L = 8, 16, 32, 64); every lane of a group gets the same bits.
template <int L>
__device__ __forceinline__ float group_sum(float x) {
  x += dpp_mov<0xb1>(x);   // quad_perm [1,0,3,2]
  x += dpp_mov<0x4e>(x);   // quad_perm [2,3,0,1]
  x += dpp_mov<0x141>(x);  // row_half_mirror: the two quads of each 8 lanes
  if constexpr (L >= 16) x += dpp_mov<0x140>(x);  // row_mirror: the two halves of each 16 lanes
  if constexpr (L >= 32) x = swap16_sum(x);
  if constexpr (L >= 64) x = swap32_sum(x);
  return x;
}

template <typename T>
__device__ __forceinline__ void ld8(const T* p, float (&x)[kVec]) {
  IO<T>::ld8(p, x);
}

template <typename T>
__device__ __forceinline__ void st8(T* p, const float (&x)[kVec]) {
  if constexpr (sizeof(T) == 2) {
    *reinterpret_cast<uint4*>(p) =
        make_uint4(pack_bf16(x[0], x[1]), pack_bf16(x[2], x[3]), pack_bf16(x[4], x[5]), pack_bf16(x[6], x[7]));
  } else {
    reinterpret_cast<float4*>(p)[0] = make_float4(x[0], x[1], x[2], x[3]);
    reinterpret_cast<float4*>(p)[1] = make_float4(x[4], x[5], x[6], x[7]);
  }
}

__device__ __forceinline__ void ld8f(const float* p, float (&x)[kVec]) { IO<float>::ld8(p, x); }

// The lane's row of D (clamped to the last one), whether it is a real row, and its first column, for the waves of
// a block taking consecutive rows from first_row, each wave `slots` groups of RPW rows (this lane's in group j).
template <int D>
struct RowLane {
  static constexpr int L = D / kVec, RPW = 64 / L;
  int64_t row;
  bool live;
  int col;
  __device__ RowLane(int64_t first_row, int64_t rows, int slots = 1, int j = 0) {
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int64_t r = first_row + (int64_t(wv) * slots + j) * RPW + lane / L;
    live = r < rows;
    row = live ? r : rows - 1;
    col = (lane % L) * kVec;
  }
};

// ---- prologue ----------------------------------------------------------------------------------------------------

// Blocks [0, nrow_blocks): rows of q_raw then k_raw (2 R rows of D), out = rnd(scale * rnd(x * rho)),
// rho = (mean(x^2) + eps)^-1/2. The blocks after them: beta and the log-decay, one (token, value head) per thread.
template <typename T, int D>
__global__ __launch_bounds__(256) void prologue_fwd_kernel(const T* __restrict__ qr, const T* __restrict__ kr,
                                                           T* __restrict__ q, T* __restrict__ k, int64_t R,
                                                           float sq, float sk, int64_t nrow_blocks,
                                                           const T* __restrict__ a, const T* __restrict__ b,
                                                           const float* __restrict__ a_log,
                                                           const float* __restrict__ dt_bias, T* __restrict__ beta,
                                                           float* __restrict__ log_decay, int64_t n, int Hv) {
  if (int64_t(blockIdx.x) >= nrow_blocks) {
    const int64_t i = (int64_t(blockIdx.x) - nrow_blocks) * 256 + threadIdx.x;
    if (i >= n) return;
    const int h = int(i % Hv);
    IO<T>::st(beta, i, gate_beta<T>(IO<T>::ld(b, i)));
    log_decay[i] = gate_log_decay<T>(IO<T>::ld(a, i), a_log[h], dt_bias[h]);
    return;
  }
  using RL = RowLane<D>;
  float x[kSlots][kVec];
  int64_t off[kSlots];
  bool isk[kSlots], live[kSlots];
#pragma unroll
  for (int j = 0; j < kSlots; ++j) {
    const RL rl(int64_t(blockIdx.x) * 4 * kSlots * RL::RPW, 2 * R, kSlots, j);
    isk[j] = rl.row >= R, live[j] = rl.live;
    off[j] = (isk[j] ? rl.row - R : rl.row) * D + rl.col;
    ld8((isk[j] ? kr : qr) + off[j], x[j]);
  }
#pragma unroll
  for (int j = 0; j < kSlots; ++j) {
    norm_row8<T>(x[j], group_sum<RL::L>(sumsq8(x[j])), D, isk[j] ? sk : sq);
    if (live[j]) st8((isk[j] ? k : q) + off[j], x[j]);
  }
}

// The backward. Row blocks: g = scale * dout, dx = rho g - rho^3 x (sum g x) / D. The blocks after them each take a
// tile of kGateSteps k tokens (k = 256 / Hv): thread t < k Hv handles value head t % Hv of tokens t / Hv,
// t / Hv + k, ..., so each step reads k Hv contiguous (token, head) elements. It writes db and da, and the tile's
// partial sums of dA_log = sum dlog_decay * log_decay and ddt_bias = sum da per head (the k threads of a head in
// order) at part[(tile * Hv + h) * 2 + {0, 1}].
template <typename T, int D>
__global__ __launch_bounds__(256) void prologue_bwd_kernel(
    const T* __restrict__ qr, const T* __restrict__ kr, const T* __restrict__ dq, const T* __restrict__ dk,
    T* __restrict__ dqr, T* __restrict__ dkr, int64_t R, float sq, float sk, int64_t nrow_blocks,
    const T* __restrict__ a, const T* __restrict__ b, const float* __restrict__ a_log,
    const float* __restrict__ dt_bias, const T* __restrict__ dbeta, const float* __restrict__ dld,
    T* __restrict__ da, T* __restrict__ db, float* __restrict__ part, int64_t BT, int Hv) {
  if (int64_t(blockIdx.x) >= nrow_blocks) {
    __shared__ float red[2][256];
    const int64_t tile = int64_t(blockIdx.x) - nrow_blocks;
    const int k = 256 / Hv, t = threadIdx.x, h = t % Hv;
    float pa = 0.f, pd = 0.f;
    if (t < k * Hv) {
      const float ea = expf(a_log[h]), bias = dt_bias[h];
      const int64_t tt = int64_t(kGateSteps) * k, end = (tile + 1) * tt < BT ? (tile + 1) * tt : BT;
      for (int64_t tok = tile * tt + t / Hv; tok < end; tok += k) {
        const int64_t i = tok * Hv + h;
        float dxa, dxb, ta, td;  // d log_decay / d A_log = log_decay
        gate_bwd<T>(IO<T>::ld(a, i), IO<T>::ld(b, i), IO<T>::ld(dbeta, i), dld[i], ea, bias, dxa, dxb, ta, td);
        IO<T>::st(db, i, dxb);
        IO<T>::st(da, i, dxa);
        pa += ta;
        pd += td;
      }
    }
    red[0][t] = pa, red[1][t] = pd;
    __syncthreads();
    if (t < Hv) {
      float sa = 0.f, sd = 0.f;
      for (int j = 0; j < k; ++j) sa += red[0][j * Hv + t], sd += red[1][j * Hv + t];
      part[(tile * Hv + t) * 2] = sa;
      part[(tile * Hv + t) * 2 + 1] = sd;
    }
    return;
  }
  using RL = RowLane<D>;
  float x[kSlots][kVec], g[kSlots][kVec];
  int64_t off[kSlots];
  bool isk[kSlots], live[kSlots];
#pragma unroll
  for (int j = 0; j < kSlots; ++j) {
    const RL rl(int64_t(blockIdx.x) * 4 * kSlots * RL::RPW, 2 * R, kSlots, j);
    isk[j] = rl.row >= R, live[j] = rl.live;
    off[j] = (isk[j] ? rl.row - R : rl.row) * D + rl.col;
    ld8((isk[j] ? kr : qr) + off[j], x[j]);
    ld8((isk[j] ? dk : dq) + off[j], g[j]);
  }
#pragma unroll
  for (int j = 0; j < kSlots; ++j) {
    float ss, gx;
    norm_bwd_sums(x[j], g[j], isk[j] ? sk : sq, ss, gx);
    norm_bwd_apply(x[j], g[j], group_sum<RL::L>(ss), group_sum<RL::L>(gx), D);
    if (live[j]) st8((isk[j] ? dkr : dqr) + off[j], x[j]);
  }
}

// ---- epilogue ----------------------------------------------------------------------------------------------------

// The gated RMSNorm: o = rnd(silu(z) * (w * (y * rho))), float32 until the one rounding (the weight is float32, so
// the rms_norm's output is; the product with silu(z) is taken in float32 and rounded once).
template <typename T, int D>
__global__ __launch_bounds__(256) void epilogue_fwd_kernel(const T* __restrict__ y, const T* __restrict__ z,
                                                           const float* __restrict__ w, float eps,
                                                           T* __restrict__ o, int64_t R) {
  using RL = RowLane<D>;
  float x[kSlots][kVec], zz[kSlots][kVec], wl[kVec];
  int64_t off[kSlots];
  bool live[kSlots];
#pragma unroll
  for (int j = 0; j < kSlots; ++j) {
    const RL rl(int64_t(blockIdx.x) * 4 * kSlots * RL::RPW, R, kSlots, j);
    live[j] = rl.live, off[j] = rl.row * D + rl.col;
    ld8(y + off[j], x[j]);
    ld8(z + off[j], zz[j]);
  }
  ld8f(w + ((threadIdx.x & 63) % RL::L) * kVec, wl);
#pragma unroll
  for (int j = 0; j < kSlots; ++j) {
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < kVec; ++e) ss += x[j][e] * x[j][e];
    const float rho = rsqrt_mean(group_sum<RL::L>(ss), D, eps);
#pragma unroll
    for (int e = 0; e < kVec; ++e) {
      const float n = wl[e] * (x[j][e] * rho);
      x[j][e] = zz[j][e] * sigmoidf(zz[j][e]) * n;
    }
    if (live[j]) st8(o + off[j], x[j]);
  }
}

// Its backward, blocks of 16 waves striding over the rows: dz = dout n silu'(z), dy through the norm, and the
// block's partial dw per column, summed in a fixed order: each lane over its rows, the wave's row slots by a
// butterfly over lanes, then the 16 waves in order.
template <typename T, int D>
__global__ __launch_bounds__(1024) void epilogue_bwd_kernel(const T* __restrict__ y, const T* __restrict__ z,
                                                            const float* __restrict__ w, float eps,
                                                            const T* __restrict__ dout, T* __restrict__ dy,
                                                            T* __restrict__ dz, float* __restrict__ part,
                                                            int64_t R) {
  using RL = RowLane<D>;
  constexpr int kRowsPerStep = 16 * RL::RPW;
  __shared__ float acc[16][D];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  float pw[kVec], wl[kVec];
  ld8f(w + (lane % RL::L) * kVec, wl);
#pragma unroll
  for (int e = 0; e < kVec; ++e) pw[e] = 0.f;
  for (int64_t first = int64_t(blockIdx.x) * kRowsPerStep; first < R; first += int64_t(gridDim.x) * kRowsPerStep) {
    const RL rl(first, R);
    const int64_t off = rl.row * D + rl.col;
    float x[kVec], zz[kVec], go[kVec];
    ld8(y + off, x);
    ld8(z + off, zz);
    ld8(dout + off, go);
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < kVec; ++e) ss += x[e] * x[e];
    const float rho = rsqrt_mean(group_sum<RL::L>(ss), D, eps);
    const float keep = rl.live ? 1.f : 0.f;
    float gx = 0.f, g[kVec];
#pragma unroll
    for (int e = 0; e < kVec; ++e) {
      const float sg = sigmoidf(zz[e]), silu = zz[e] * sg, nh = x[e] * rho;
      zz[e] = go[e] * nh * wl[e] * sg * (1.f + zz[e] * (1.f - sg));  // dz
      const float dn = go[e] * silu;
      pw[e] += keep * (dn * nh);
      g[e] = dn * wl[e];
      gx += g[e] * x[e];
    }
    const float c = rho * rho * rho * group_sum<RL::L>(gx) / D;
#pragma unroll
    for (int e = 0; e < kVec; ++e) x[e] = rho * g[e] - c * x[e];
    if (rl.live) {
      st8(dz + off, zz);
      st8(dy + off, x);
    }
  }
#pragma unroll
  for (int e = 0; e < kVec; ++e) {  // the sum over the wave's row slots: lanes l ^ L, l ^ 2L, ...
    if constexpr (RL::L < 16) pw[e] += __shfl_xor(pw[e], 8);
    if constexpr (RL::L < 32) pw[e] = swap16_sum(pw[e]);
    pw[e] = swap32_sum(pw[e]);
  }
  if (lane < RL::L) {
#pragma unroll
    for (int e = 0; e < kVec; ++e) acc[wv][lane * kVec + e] = pw[e];
  }
  __syncthreads();
  if (threadIdx.x < D) {
    float s = 0.f;
#pragma unroll
    for (int v = 0; v < 16; ++v) s += acc[v][threadIdx.x];
    part[int64_t(blockIdx.x) * D + threadIdx.x] = s;
  }
}

// Sums of partials: column c < width of out is the sum over parts p of part[p * width + c], in a fixed order (64
// columns per block, wave v summing the parts p = v mod 16 in increasing order, then the 16 waves in order). With
// `pairs`, columns alternate between two outputs: column 2 h + j goes to out_j[h].
template <bool pairs>
__global__ __launch_bounds__(1024) void sum_parts(const float* __restrict__ part, int64_t nparts, int width,
                                                  float* __restrict__ out0, float* __restrict__ out1) {
  __shared__ float red[16][64];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int c = blockIdx.x * 64 + lane;
  float s = 0.f;
  if (c < width)
    for (int64_t p0 = wv; p0 < nparts; p0 += 16 * 16) {  // 16 loads in flight, then summed in order
      float v[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int64_t p = p0 + 16 * i;
        v[i] = p < nparts ? part[p * width + c] : 0.f;
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) s += v[i];
    }
  red[wv][lane] = s;
  __syncthreads();
  if (wv == 0 && c < width) {
    float t = 0.f;
#pragma unroll
    for (int v = 0; v < 16; ++v) t += red[v][lane];
    if constexpr (pairs)
      ((c & 1) ? out1 : out0)[c >> 1] = t;
    else
      out0[c] = t;
  }
}

}  // namespace

// Host side -------------------------------------------------------------------------------------------------------

namespace {

template <int D>
constexpr int64_t rows_per_block() {
  return 4 * kSlots * RowLane<D>::RPW;
}

int64_t gate_tiles(int64_t BT, int Hv) {
  const int64_t tt = int64_t(kGateSteps) * (256 / Hv);
  return (BT + tt - 1) / tt;
}

template <int D>
int64_t norm_bwd_blocks(int64_t R) {
  const int64_t steps = (R + 16 * RowLane<D>::RPW - 1) / (16 * RowLane<D>::RPW);
  return steps < kNormBwdBlocks ? steps : kNormBwdBlocks;
}

int64_t norm_bwd_blocks_of(int D, int64_t R) {
  switch (D) {
    case 64: return norm_bwd_blocks<64>(R);
    case 128: return norm_bwd_blocks<128>(R);
    default: return norm_bwd_blocks<256>(R);
  }
}

template <int D, typename T>
hipError_t prologue_fwd_d(const NbProblem& p, const NbPrologue& x, hipStream_t s) {
  const int64_t R = p.BT * p.Hk, n = p.BT * p.Hv;
  const int64_t row_blocks = (2 * R + rows_per_block<D>() - 1) / rows_per_block<D>();
  const int64_t blocks = row_blocks + (n + 255) / 256;
  if (blocks)
    hipLaunchKernelGGL((prologue_fwd_kernel<T, D>), dim3(unsigned(blocks)), dim3(256), 0, s,
                       static_cast<const T*>(x.q_raw), static_cast<const T*>(x.k_raw), static_cast<T*>(x.q),
                       static_cast<T*>(x.k), R, p.scale_q, p.scale_k, row_blocks, static_cast<const T*>(x.a),
                       static_cast<const T*>(x.b), x.a_log, x.dt_bias, static_cast<T*>(x.beta), x.log_decay, n,
                       p.Hv);
  return hipGetLastError();
}

template <int D, typename T>
hipError_t prologue_bwd_d(const NbProblem& p, const NbPrologueGrad& x, void* ws, hipStream_t s) {
  const int64_t R = p.BT * p.Hk, tiles = gate_tiles(p.BT, p.Hv);
  const int64_t row_blocks = (2 * R + rows_per_block<D>() - 1) / rows_per_block<D>();
  const int64_t blocks = row_blocks + tiles;
  float* part = static_cast<float*>(ws);
  if (blocks)
    hipLaunchKernelGGL((prologue_bwd_kernel<T, D>), dim3(unsigned(blocks)), dim3(256), 0, s,
                       static_cast<const T*>(x.q_raw), static_cast<const T*>(x.k_raw), static_cast<const T*>(x.dq),
                       static_cast<const T*>(x.dk), static_cast<T*>(x.dq_raw), static_cast<T*>(x.dk_raw), R,
                       p.scale_q, p.scale_k, row_blocks, static_cast<const T*>(x.a), static_cast<const T*>(x.b),
                       x.a_log, x.dt_bias, static_cast<const T*>(x.dbeta), x.dlog_decay, static_cast<T*>(x.da),
                       static_cast<T*>(x.db), part, p.BT, p.Hv);
  // (With no tokens, sums over no parts: zeros.)
  hipLaunchKernelGGL(sum_parts<true>, dim3(unsigned((2 * p.Hv + 63) / 64)), dim3(1024), 0, s, part, tiles,
                     2 * p.Hv, x.da_log, x.ddt_bias);
  return hipGetLastError();
}

template <int D, typename T>
hipError_t epilogue_fwd_d(const NbProblem& p, const NbEpilogue& x, hipStream_t s) {
  const int64_t R = p.BT * p.Hv;
  const int64_t blocks = (R + rows_per_block<D>() - 1) / rows_per_block<D>();
  if (blocks)
    hipLaunchKernelGGL((epilogue_fwd_kernel<T, D>), dim3(unsigned(blocks)), dim3(256), 0, s,
                       static_cast<const T*>(x.y), static_cast<const T*>(x.z), x.w, x.eps, static_cast<T*>(x.o), R);
  return hipGetLastError();
}

template <int D, typename T>
hipError_t epilogue_bwd_d(const NbProblem& p, const NbEpilogueGrad& x, void* ws, hipStream_t s) {
  const int64_t R = p.BT * p.Hv;
  const int64_t blocks = norm_bwd_blocks<D>(R);
  float* part = static_cast<float*>(ws);
  if (blocks)
    hipLaunchKernelGGL((epilogue_bwd_kernel<T, D>), dim3(unsigned(blocks)), dim3(1024), 0, s,
                       static_cast<const T*>(x.y), static_cast<const T*>(x.z), x.w, x.eps,
                       static_cast<const T*>(x.dout), static_cast<T*>(x.dy), static_cast<T*>(x.dz), part, R);
  // (With no rows, a sum over no parts: zeros.)
  hipLaunchKernelGGL(sum_parts<false>, dim3(unsigned((D + 63) / 64)), dim3(1024), 0, s, part, blocks, D, x.dw,
                     nullptr);
  return hipGetLastError();
}

template <typename F>
hipError_t by_width(int D, F&& f) {
  switch (D) {
    case 64: return f(std::integral_constant<int, 64>{});
    case 128: return f(std::integral_constant<int, 128>{});
    case 256: return f(std::integral_constant<int, 256>{});
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

const char* nb_supports(const NbProblem& p, bool uses_dk, bool uses_dv) {
  auto ok = [](int D) { return D == 64 || D == 128 || D == 256; };
  if (uses_dk && !ok(p.Dk)) return "the neighbour kernels need Dk of 64, 128 or 256";
  if (uses_dv && !ok(p.Dv)) return "the neighbour kernels need Dv of 64, 128 or 256";
  if (!uses_dk && !uses_dv && !ok(p.Dk) && !ok(p.Dv)) return "the neighbour kernels need Dk or Dv of 64, 128 or 256";
  if (p.Hv > 256) return "the neighbour kernels need at most 256 value heads";
  return nullptr;
}

size_t nb_workspace_bytes(const NbProblem& p) {
  const size_t gates = size_t(gate_tiles(p.BT, p.Hv)) * p.Hv * 2 * 4;
  const size_t norm = size_t(norm_bwd_blocks_of(p.Dv, p.BT * p.Hv)) * p.Dv * 4;
  return gates > norm ? gates : norm;
}

hipError_t nb_prologue_fwd(const NbProblem& p, const NbPrologue& x, hipStream_t s) {
  return by_width(p.Dk, [&](auto dc) {
    constexpr int D = decltype(dc)::value;
    return p.bf16 ? prologue_fwd_d<D, bf16_t>(p, x, s) : prologue_fwd_d<D, float>(p, x, s);
  });
}

hipError_t nb_prologue_bwd(const NbProblem& p, const NbPrologueGrad& x, void* ws, hipStream_t s) {
  return by_width(p.Dk, [&](auto dc) {
    constexpr int D = decltype(dc)::value;
    return p.bf16 ? prologue_bwd_d<D, bf16_t>(p, x, ws, s) : prologue_bwd_d<D, float>(p, x, ws, s);
  });
}

hipError_t nb_epilogue_fwd(const NbProblem& p, const NbEpilogue& x, hipStream_t s) {
  return by_width(p.Dv, [&](auto dc) {
    constexpr int D = decltype(dc)::value;
    return p.bf16 ? epilogue_fwd_d<D, bf16_t>(p, x, s) : epilogue_fwd_d<D, float>(p, x, s);
  });
}

hipError_t nb_epilogue_bwd(const NbProblem& p, const NbEpilogueGrad& x, void* ws, hipStream_t s) {
  return by_width(p.Dv, [&](auto dc) {
    constexpr int D = decltype(dc)::value;
    return p.bf16 ? epilogue_bwd_d<D, bf16_t>(p, x, ws, s) : epilogue_bwd_d<D, float>(p, x, ws, s);
  });
}

}  // namespace qbgdn
