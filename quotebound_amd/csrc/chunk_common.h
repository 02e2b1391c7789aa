// Shared pieces of the chunked design: buffer layouts, the chunk-slot -> (sequence, chunk) map, and staging.
//
// Residuals (the ckpt buffer): the chunk-start states, then per chunk slot s and value head h a Tile record that
// the prep kernel writes and the other three kernels read:
//   states  [NC][Hv][Dv][Dk]  f32   state at the chunk's start (the reference's ckpt, src/delta_grad.cpp:172-181)
//   tiles   [NC][Hv] Tile
// Workspace: dSend [NC][Hv][Dv][Dk] f32, the cotangent of the state at each chunk's end.
#pragma once
#include "gdn_common.h"
#include "mfma.h"

namespace qbgdn {

constexpr int kC = kChunk;  // 64 positions per chunk
constexpr int kPadB = 8;    // bf16 row padding in LDS (keeps 16-byte alignment, staggers banks)

// Everything about a (chunk, value head) that does not depend on the state, as MFMA-ready bf16 hi/lo pairs:
//   T = (I + A)^-1, A = strict_lower(diag(beta) (E * K K^T)), E_ij = exp(G_i - G_j)
//   P = lower_incl(E * Q K^T)
// and the per-position vectors. Positions past the chunk's end are padded (beta 0, log-decay 0, k = q = 0).
// Every step's delta_t of the chunk is T diag(beta) R; the readers apply beta to R's rows (and to the rows of dR in
// the backward) rather than keep T diag(beta) as a third matrix. The two 64 x 64 matrices are lower triangular; each
// is stored as its ten 16 x 16 blocks on or below the diagonal (tri_off), so the record holds no zero blocks.
constexpr int kTri = 10 * 256;

// Element offset of (i, j), j / 16 <= i / 16, in a lower-triangular 64 x 64 matrix stored as the blocks (I, J),
// J <= I, in the order (0,0) (1,0) (1,1) (2,0) .. (3,3), each row-major: a row of a block is 16 contiguous
// elements (32 bytes), and the blocks (I, 0..I) of a row strip are contiguous.
__host__ __device__ constexpr int tri_off(int i, int j) {
  return (((i >> 4) * ((i >> 4) + 1) / 2 + (j >> 4)) << 8) + ((i & 15) << 4) + (j & 15);
}

struct Tile {
  bf16_t t[2][kTri];  // T, hi and lo (row i, column j)
  bf16_t p[2][kTri];  // P, hi and lo (row i: query, column j: key)
  float gam[kC];      // exp(G_i)
  float dec[kC];      // exp(G_63 - G_i)
  float beta[kC];
  float G[kC];        // G_i = sum_{j <= i} a_j within the chunk
};
static_assert(sizeof(Tile) % 16 == 0, "Tile records stay 16-byte aligned");

// Eight bf16 of row i, columns c .. c + 7 (c a multiple of 8), of the packed triangular matrix whose hi half starts
// at element h0 of the buffer resource r (lo at h0 + kTri); groups in a block above the diagonal read zeros (their
// offset lies past the resource).
__device__ __forceinline__ bf16x8 tri_ld8(__amdgpu_buffer_rsrc_t r, int h0, int i, int c) {
  const uint32_t off = (c >> 4) <= (i >> 4) ? uint32_t(h0 + tri_off(i, c)) * 2u : 0x80000000u;
  return __builtin_bit_cast(bf16x8, buf_ld16(r, off));
}

// The MFMA operand whose k index runs down the rows of a packed lower-triangular matrix M held in LDS (tri_off
// layout, M at element 0): lane (g = lane / 16, n = lane % 16) gets M[r0 + 8g + jj][16 J + n], jj = 0..7, for a
// multiple r0 of 32. Each lane supplies its own addresses to gfx950's transposing LDS read (four consecutive
// columns of one row are contiguous in a block); the rows 8g .. 8g + 7 lie in one block, and a block above the
// diagonal reads zeros.
__device__ __forceinline__ bf16x8 tri_tr8(const __bf16* M, int r0, int J, int lane) {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
  const int s = lane & 15, g = (lane >> 4) & 3, ra = r0 + 8 * g + (s >> 2), c = 16 * J + 4 * (s & 3);
  const bool in = (ra >> 4) >= J;
  const s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(M + (in ? tri_off(ra, c) : 0)));
  const s16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(M + (in ? tri_off(ra + 4, c) : 0)));
  const bf16x4 x = __builtin_bit_cast(bf16x4, a), y = __builtin_bit_cast(bf16x4, b);
  const bf16x8 v = __builtin_shufflevector(x, y, 0, 1, 2, 3, 4, 5, 6, 7);
  const bf16x8 z = {};
  return in ? v : z;
}

struct ChunkLayout {
  int64_t NC;
  int Hv, Dv, Dk;
  __host__ __device__ int64_t states_elems() const { return NC * Hv * int64_t(Dv) * Dk; }
  __host__ __device__ size_t tiles_bytes() const { return size_t(NC) * Hv * sizeof(Tile); }
  __host__ __device__ size_t bytes() const { return size_t(states_elems()) * 4 + tiles_bytes(); }
};

// The sequence and chunk of a chunk slot (slots of sequence n are [slot0[n], slot0[n + 1])).
struct SlotPos {
  int n, c;
  int64_t tok;  // first token of the chunk
  int L;        // valid positions
};

__device__ __forceinline__ SlotPos slot_pos(const SeqTable& tab, int64_t slot) {
  int n, c;
  if (tab.n == 0) {
    n = int(slot / tab.nc);
    c = int(slot - int64_t(n) * tab.nc);
  } else {  // largest n with slot0[n] <= slot (empty sequences share a slot0 with their successor)
    int lo = 0, hi = tab.n - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (tab.slot0[mid] <= slot) lo = mid; else hi = mid - 1;
    }
    n = lo;
    c = int(slot - tab.slot0[n]);
  }
  const Seq sq = seq_of(tab, n);
  const int t0 = c * kC;
  return SlotPos{n, c, sq.tok0 + t0, min(kC, sq.len - t0)};
}

// Four consecutive values at element offset at (a multiple of 4) of the hi and lo matrices, as bf16 hi/lo halves.
__device__ __forceinline__ void put4(__bf16* hi, __bf16* lo, int at, float x0, float x1, float x2, float x3) {
  const Split4 v = split4(x0, x1, x2, x3);
  *reinterpret_cast<uint2*>(hi + at) = v.hi;
  *reinterpret_cast<uint2*>(lo + at) = v.lo;
}
__device__ __forceinline__ void put4(__bf16* hi, __bf16* lo, int at, const f32x4& x) {
  put4(hi, lo, at, x[0], x[1], x[2], x[3]);
}

// Copies rows [0, L) of a [tokens, H, D] bf16 tensor's head h into LDS rows of length D (stride ld), zero rows past
// L. 8 elements per access.
template <int D>
__device__ __forceinline__ void stage_rows_bf16(__bf16* dst, int ld, const bf16_t* src, int64_t tok, int H, int h,
                                                int L, int nthreads) {
  constexpr int V8 = D / 8;
  for (int e = threadIdx.x; e < kC * V8; e += nthreads) {
    const int t = e / V8, c8 = (e % V8) * 8;
    bf16x8 v;
    if (t < L) {
      v = gld8(src + ((tok + t) * H + h) * int64_t(D) + c8);
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = (__bf16)0.f;
    }
    *reinterpret_cast<bf16x8*>(dst + t * ld + c8) = v;
  }
}

// The decay factor's log: the input itself (g_is_log) or log of the factor.
__device__ __forceinline__ double log_decay(const float* g, int64_t i, int g_is_log) {
  const float x = g[i];
  return g_is_log ? double(x) : log(double(x));
}

}  // namespace qbgdn
