// Device-side pieces shared by both designs: element I/O for float32 and bfloat16, wave64 lane reductions, and the
// table that maps a (sequence, step) to its token and chunk slot.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qbgdn {

constexpr int kChunk = 64;     // checkpoint stride, the reference's kChunk (src/delta_grad.cpp:11)
constexpr int kMaxSeqs = 255;  // packed sequences per call

// bfloat16 is carried as its bit pattern.
typedef uint16_t bf16_t;

__device__ __forceinline__ float bf16_to_f32(bf16_t b) { return __uint_as_float(uint32_t(b) << 16); }

// Two floats to packed bf16 (x0 in the low half), rounded to nearest even, NaN staying NaN: one
// v_cvt_pk_bf16_f32.
__device__ __forceinline__ uint32_t f32x2_to_bf16x2(float x0, float x1) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{x0, x1}, bf16x2_t));
}
__device__ __forceinline__ bf16_t f32_to_bf16(float f) { return bf16_t(f32x2_to_bf16x2(f, 0.f)); }

template <typename T>
struct IO;
template <>
struct IO<float> {
  static __device__ __forceinline__ float ld(const float* p, int64_t i) { return p[i]; }
  static __device__ __forceinline__ void st(float* p, int64_t i, float x) { p[i] = x; }
  // 8 consecutive elements from a 16-byte aligned address.
  static __device__ __forceinline__ void ld8(const float* p, float* o) {
    const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
    o[0] = a.x, o[1] = a.y, o[2] = a.z, o[3] = a.w, o[4] = b.x, o[5] = b.y, o[6] = b.z, o[7] = b.w;
  }
};
template <>
struct IO<bf16_t> {
  static __device__ __forceinline__ float ld(const bf16_t* p, int64_t i) { return bf16_to_f32(p[i]); }
  static __device__ __forceinline__ void st(bf16_t* p, int64_t i, float x) { p[i] = f32_to_bf16(x); }
  static __device__ __forceinline__ void ld8(const bf16_t* p, float* o) {
    const uint4 r = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[2 * i] = __uint_as_float(w[i] << 16);
      o[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
};

// ---- buffer stores -----------------------------------------------------------------------------------------------
// A raw buffer resource over [base, base + bytes): vector stores at byte offsets past the range are dropped by the
// hardware. Masked stores of a tile's last rows then need no branch, which keeps the compiler's count of outstanding
// memory operations exact (a branch around a store makes it wait for every load in flight). bytes == 0 drops every
// store. Word 3 is the untyped-buffer format word of CDNA (32-bit data format).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, int(bytes), 0x00020000);
}
// Loads at byte offsets past the range return zeros.
__device__ __forceinline__ uint4 buf_ld16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, int(byte_off), 0, 0);
  return uint4{v[0], v[1], v[2], v[3]};
}
// Stores at byte offsets past the range are dropped.
__device__ __forceinline__ void buf_st16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off, uint4 v) {
  typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4;
  __builtin_amdgcn_raw_buffer_store_b128(u32x4{v.x, v.y, v.z, v.w}, r, int(byte_off), 0, 0);
}
__device__ __forceinline__ uint2 buf_ld8(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, int(byte_off), 0, 0);
  return uint2{v[0], v[1]};
}
__device__ __forceinline__ uint16_t buf_ld2(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, int(byte_off), 0, 0);
}
__device__ __forceinline__ float buf_ld4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, int(byte_off), 0, 0));
}

template <typename T>
struct BufIO;
template <>
struct BufIO<float> {
  static __device__ __forceinline__ void st(__amdgpu_buffer_rsrc_t r, uint32_t i, float x) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(x), r, int(i * 4), 0, 0);
  }
  // Elements i .. i + 3 (i a multiple of 4) in one 16-byte store.
  template <typename V4>
  static __device__ __forceinline__ void st4(__amdgpu_buffer_rsrc_t r, uint32_t i, const V4& x) {
    typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4;
    const u32x4 v = {__float_as_uint(x[0]), __float_as_uint(x[1]), __float_as_uint(x[2]), __float_as_uint(x[3])};
    __builtin_amdgcn_raw_buffer_store_b128(v, r, int(i * 4), 0, 0);
  }
};
template <>
struct BufIO<bf16_t> {
  static __device__ __forceinline__ void st(__amdgpu_buffer_rsrc_t r, uint32_t i, float x) {
    __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16(x), r, int(i * 2), 0, 0);
  }
  // Elements i .. i + 3 (i a multiple of 4) in one 8-byte store.
  template <typename V4>
  static __device__ __forceinline__ void st4(__amdgpu_buffer_rsrc_t r, uint32_t i, const V4& x) {
    typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u32x2;
    const u32x2 v = {f32x2_to_bf16x2(x[0], x[1]), f32x2_to_bf16x2(x[2], x[3])};
    __builtin_amdgcn_raw_buffer_store_b64(v, r, int(i * 2), 0, 0);
  }
};

// ---- lane reductions ------------------------------------------------------------------------------------------
// DPP controls (gfx9 encoding): quad_perm, row_mirror, row_half_mirror.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}

// Sum over each 16-lane row of the wave; every lane of the row gets the same bits (each stage pairs lanes
// symmetrically, and a + b == b + a).
__device__ __forceinline__ float sum16(float x) {
  x += dpp_mov<0xb1>(x);   // quad_perm [1,0,3,2]
  x += dpp_mov<0x4e>(x);   // quad_perm [2,3,0,1]
  x += dpp_mov<0x141>(x);  // row_half_mirror: quad q pairs with quad q^1
  x += dpp_mov<0x140>(x);  // row_mirror: half-row h pairs with h^1
  return x;
}

// x plus x of lane ^ 16 (swap16_sum) or lane ^ 32 (swap32_sum), each one gfx950 lane swap and an add, no LDS:
// v_permlane16_swap(x, x) leaves (x, x of lane + 16) in the low 16 lanes of every 32 and (x of lane - 16, x) in the
// high ones (v_permlane32_swap likewise for the two 32-lane halves), so the two lanes of a pair add the same two
// values and, addition being commutative, get the same bits as x + __shfl_xor(x, 16 or 32) would give.
__device__ __forceinline__ float swap16_sum(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float swap32_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// The sums of a and of b over each group of 32 lanes, both given to every lane of the group, on one 16-lane DPP
// tree: v_permlane16_swap(a, b) plus an add leaves a + (a of lane + 16) in the low 16 lanes of every 32 and
// (b of lane - 16) + b in the high ones; sum16 finishes a's sum in the low lanes and b's in the high; a second swap
// of that value with itself hands each half the other's (first result: a's sum everywhere, second: b's).
__device__ __forceinline__ void sum32_pair(float& a, float& b) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  const float x = sum16(__uint_as_float(r[0]) + __uint_as_float(r[1]));
  const auto t = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  a = __uint_as_float(t[0]);
  b = __uint_as_float(t[1]);
}

// Blocks are dispatched round-robin over the MI355X's 8 XCDs (block id runs on XCD id % 8), each with its own
// L2. This gives XCD x a contiguous range of work items, so neighbouring items (which read the same key head)
// share an L2. A bijection on [0, n).
__device__ __forceinline__ int xcd_remap(int id, int n) {
  const int per = n >> 3, rem = n & 7;
  const int x = id & 7, s = id >> 3;
  return x * per + (x < rem ? x : rem) + s;
}

// ---- packed sequences ------------------------------------------------------------------------------------------
// Passed by value as a kernel argument. n == 0: batch mode, sequence i is batch row i (T tokens, nc chunk slots
// each). n > 0: tok0[i] is the first token of sequence i (tok0[n] == total tokens) and slot0[i] its first chunk
// slot (slot0[n] == total slots).
struct SeqTable {
  int32_t n;
  int32_t T;
  int32_t nc;
  int32_t tok0[kMaxSeqs + 1];
  int32_t slot0[kMaxSeqs + 1];
  uint8_t longest[kMaxSeqs];  // n > 0: the sequences by decreasing length (ties by index)
};

struct Seq {
  int64_t tok0;  // flattened index of the first token in [B * T]
  int32_t len;   // steps
  int64_t slot0; // first chunk slot
};

__device__ __forceinline__ Seq seq_of(const SeqTable& tab, int i) {
  if (tab.n == 0) return Seq{int64_t(i) * tab.T, tab.T, int64_t(i) * tab.nc};
  return Seq{tab.tok0[i], tab.tok0[i + 1] - tab.tok0[i], tab.slot0[i]};
}

// The work item of block `id` in the passes that walk a sequence's chunks in order (the state passes, the
// recurrent design): row block `blk` of value head `hv` of sequence `n`, among total = nblk * Hv * N items. The
// items of one (sequence, key head) form a group of G = nblk * (Hv / Hk) blocks reading the same q and k rows.
// Batch mode: XCD x takes a contiguous range of items (xcd_remap), so groups stay on one XCD. Packed mode: the
// groups, longest sequence first, are dealt to the XCDs in turn, every block of a group on one XCD (blocks id,
// id + 8, id + 16, ... run on XCD id % 8). Long sequences start first and every XCD gets its share of each length,
// where a contiguous range would give one XCD the longest sequence's every item. A bijection on [0, total).
struct StateItem {
  int blk, hv, n;
};
__device__ __forceinline__ StateItem state_item(const SeqTable& tab, int id, int nblk, int Hv, int Hk, int total) {
  if (tab.n == 0) {
    const int w = xcd_remap(id, total);
    return StateItem{w % nblk, (w / nblk) % Hv, w / (nblk * Hv)};
  }
  const int per_hk = Hv / Hk, G = nblk * per_hk, ngroups = total / G, full = ngroups >> 3;
  int rank, j;  // the group's place in the order, the item within the group
  const int sb = id / (8 * G);
  if (sb < full) {  // 8 whole groups, group 8 sb + x on XCD x
    const int t = id - sb * 8 * G;
    rank = 8 * sb + (t & 7), j = t >> 3;
  } else {  // the last 1..7 groups
    const int rest = ngroups - 8 * full, t = id - full * 8 * G;
    rank = 8 * full + t % rest, j = t / rest;
  }
  return StateItem{j % nblk, (rank % Hk) * per_hk + j / nblk, int(tab.longest[rank / Hk])};
}

}  // namespace qbgdn
