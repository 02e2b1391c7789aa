// MFMA building blocks for the chunked design: v_mfma_f32_16x16x32_bf16 (gfx950) with float32 operands split
// into a bf16 pair (hi = rne(x), lo = rne(x - hi)) so products of float32 values keep ~2^-16 relative accuracy:
//   x * y ~= hi(x) hi(y) + hi(x) lo(y) + lo(x) hi(y)        (three MFMAs; two when one side is exact in bf16).
//
// Lane layouts of v_mfma_f32_16x16x32_bf16 (wave64, lane l, g = l / 16):
//   A [16 x 32]: lane l holds row l % 16, k = 8 g + 0..7
//   B [32 x 16]: lane l holds col l % 16, k = 8 g + 0..7
//   C [16 x 16]: lane l holds col l % 16, rows 4 g + 0..3
// The contraction index k may be permuted freely as long as A and B use the same permutation. Two stacked C tiles
// (rows 0-15 and 16-31 of a 32-row block) therefore feed a later product directly as its k = 32 operand with
// k order {4g + 0..3, 16 + 4g + 0..3}: a C result can be used, without moving it, as the operand that contracts
// over C's row index. kperm() gives that order.
#pragma once
#include <hip/hip_runtime.h>

#include "gdn_common.h"

namespace qbgdn {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;

__device__ __forceinline__ f32x4 mma(f32x4 c, bf16x8 a, bf16x8 b) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

struct Split8 {
  bf16x8 hi, lo;
};

typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
typedef float f32x2v __attribute__((ext_vector_type(2)));

// x0, x1 as packed bf16 pairs hi = rne(x) and lo = rne(x - hi) (x = hi + lo to about 16 bits): two values per
// v_cvt_pk_bf16_f32, so neither pair needs packing, and hi widens back to float by a shift or a mask.
__device__ __forceinline__ void split2(float x0, float x1, uint32_t& hi, uint32_t& lo) {
  hi = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2v{x0, x1}, bf16x2v));
  const float h0 = __uint_as_float(hi << 16), h1 = __uint_as_float(hi & 0xffff0000u);
  lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2v{x0 - h0, x1 - h1}, bf16x2v));
}

__device__ __forceinline__ Split8 split8(const float* x) {
  uint4 h, l;
  split2(x[0], x[1], h.x, l.x);
  split2(x[2], x[3], h.y, l.y);
  split2(x[4], x[5], h.z, l.z);
  split2(x[6], x[7], h.w, l.w);
  return Split8{__builtin_bit_cast(bf16x8, h), __builtin_bit_cast(bf16x8, l)};
}

// acc += A * B for split operands (three MFMAs).
__device__ __forceinline__ f32x4 mma3(f32x4 c, const Split8& a, const Split8& b) {
  c = mma(c, a.hi, b.hi);
  c = mma(c, a.hi, b.lo);
  return mma(c, a.lo, b.hi);
}
// acc += A * B with B exact in bf16 (two MFMAs).
__device__ __forceinline__ f32x4 mma2(f32x4 c, const Split8& a, bf16x8 b) {
  c = mma(c, a.hi, b);
  return mma(c, a.lo, b);
}
__device__ __forceinline__ f32x4 mma2(f32x4 c, bf16x8 a, const Split8& b) {
  c = mma(c, a, b.hi);
  return mma(c, a, b.lo);
}

__device__ __forceinline__ f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

// Position of element j (0..7) of a lane in k group g under the stacked-C order: {4g + 0..3, 16 + 4g + 0..3}.
__device__ __forceinline__ int kperm(int g, int j) { return (j < 4 ? 4 * g + j : 16 + 4 * g + (j - 4)); }

// Loads 8 consecutive bf16 from LDS (16-byte aligned).
__device__ __forceinline__ bf16x8 lds8(const __bf16* p) { return *reinterpret_cast<const bf16x8*>(p); }

// Loads 4 + 4 bf16 (two 8-byte runs) from LDS: p[0..3] and p[16..19], the stacked-C k order.
__device__ __forceinline__ bf16x8 lds4x2(const __bf16* p) {
  typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
  const bf16x4 a = *reinterpret_cast<const bf16x4*>(p);
  const bf16x4 b = *reinterpret_cast<const bf16x4*>(p + 16);
  return bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// Global bf16 bits -> bf16x8 (16-byte aligned).
__device__ __forceinline__ bf16x8 gld8(const bf16_t* p) { return *reinterpret_cast<const bf16x8*>(p); }

// An MFMA operand whose k index runs down the rows of a row-major bf16 LDS matrix: lane (g = lane / 16,
// n = lane % 16) gets M[8g + j][n], j = 0..7, of the matrix M at L (L points at its element [0][0]; ld, the row
// stride in elements, and the offset of L are multiples of 4). This is the operand for k = rows, n = columns (B), or
// m = columns, k = rows (A). It uses gfx950's transposing LDS read (ds_read_b64_tr_b16): within each group of 16
// lanes, lane s supplies the address of row s / 4, columns 4 (s % 4) .. + 3, and lane 4a + b receives element b
// of the rows supplied by lanes a, 4 + a, 8 + a, 12 + a. Two reads cover k = 8g .. 8g + 3 and 8g + 4 .. 8g + 7.
__device__ __forceinline__ bf16x8 lds_tr8(const __bf16* L, int ld, int lane) {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  const int s = lane & 15, g = (lane >> 4) & 3;
  const __bf16* p = L + (8 * g + (s >> 2)) * ld + 4 * (s & 3);
  typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
  const s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p));
  const s16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p + 4 * ld));
  // Whole vectors are bit-cast: a bit cast of a single vector element reads element 0 with this compiler.
  const bf16x4 x = __builtin_bit_cast(bf16x4, a), y = __builtin_bit_cast(bf16x4, b);
  return __builtin_shufflevector(x, y, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Bank-conflict-free placement of a bf16 LDS matrix whose row pitch ld is an odd multiple of 16 elements (32 bytes
// times an odd number): element (r, c) lives at swz(r, c, ld). Row r takes the slot of row r ^ 4 when bit 3 of r is
// set (rows 8-11 and 12-15 of every 16 trade places), and bit 3 of the column flips with bit 3 of the row (the two
// 16-byte halves of every 32 bytes trade places). On gfx950 (measured: 16-byte reads are served 16 lanes at a time,
// lanes 0-31 and 32-63 apart with lanes whose index bits 2-4 have equal parity together; 8-byte and transposing
// reads 32 lanes at a time; 64 banks of 4 bytes), this makes lds8 of 16 rows at k = 8g, lds_tr8s, and 16-byte row
// stores conflict-free, while a padded row-major layout leaves the transposing read 2-way conflicted for every odd
// pitch. Offsets that are multiples of 16 in both the row and the column commute with swz, so a matrix view
// L + swz(R0, C0, ld) with R0 % 16 == 0 and C0 % 16 == 0 is again swz-placed.
__device__ __forceinline__ int swz(int r, int c, int ld) { return (r ^ ((r >> 1) & 4)) * ld + (c ^ (r & 8)); }

// lds_tr8 for a swz-placed matrix: lane (g, n) gets M[8g + j][n], j = 0..7.
__device__ __forceinline__ bf16x8 lds_tr8s(const __bf16* L, int ld, int lane) {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  const int s = lane & 15, g = (lane >> 4) & 3, r = 8 * g + (s >> 2), c = 4 * (s & 3);
  typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
  const s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(L + swz(r, c, ld)));
  const s16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(L + swz(r + 4, c, ld)));
  const bf16x4 x = __builtin_bit_cast(bf16x4, a), y = __builtin_bit_cast(bf16x4, b);
  return __builtin_shufflevector(x, y, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Four consecutive values as bf16 hi and lo halves (x = hi + lo to about 16 bits), each packed into 8 bytes.
struct Split4 {
  uint2 hi, lo;
};
__device__ __forceinline__ Split4 split4(float x0, float x1, float x2, float x3) {
  Split4 s;
  split2(x0, x1, s.hi.x, s.lo.x);
  split2(x2, x3, s.hi.y, s.lo.y);
  return s;
}

}  // namespace qbgdn
